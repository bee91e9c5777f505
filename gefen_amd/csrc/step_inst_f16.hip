// Kernel instances of the Gefen step, GefenMuon momentum and packed-index
// kernels for f16 parameters, f16 state (one file per dtype pair, compiled in parallel).
#include "step_kernels.h"

namespace gefen {
GEFEN_STEP_INSTANCES(template, f16_t, f16_t)
}  // namespace gefen
