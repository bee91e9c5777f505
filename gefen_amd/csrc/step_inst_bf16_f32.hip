// Kernel instances of the Gefen step, GefenMuon momentum and packed-index
// kernels for bf16 parameters, float state (one file per dtype pair, compiled in parallel).
#include "step_kernels.h"

namespace gefen {
GEFEN_STEP_INSTANCES(template, bf16_t, float)
}  // namespace gefen
