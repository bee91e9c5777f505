"""Build libgefen_hip.so (the C-ABI library), libgefen_synth.so, the host
extension _gefen_host and the GPU tests' HIP helpers (tests/hip) in-tree.

    python -m gefen_amd.build [--jobs N]

hipcc cross-compiles for gfx950 without a GPU.  Flags:
  -ffp-contract=off        only the fused multiply-adds written in the source
                           are fused (the reference CPU path rounds every op);
  -packed-fp32-ops off     no v_pk_*_f32 code generation.
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("GEFEN_OFFLOAD_ARCH", "gfx950")

COMMON = [
    "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
    "-I", str(REPO / "include"), "-I", str(CSRC),
]

LIBS = {
    "libgefen_hip.so": ["capi.cpp", "step.hip", "step_inst_bf16.hip", "step_inst_f16.hip", "step_inst_f32.hip",
                        "step_inst_bf16_f32.hip", "step_inst_f16_f32.hip", "codebook.hip", "period.hip", "ns_gemm.hip",
                        "muon.hip"],
    "libgefen_synth.so": ["capi.cpp", "synthetic.hip"],
}


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC] + COMMON + ["-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [HIPCC] + COMMON + ["-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed on {}".format(src.name))
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (r.stdout + r.stderr).splitlines() if ln.strip() and noise not in ln]
    if msgs:
        sys.stderr.write("\n".join(msgs) + "\n")


def _stale(src: Path, obj: Path) -> bool:
    """obj is older than src or than any header of csrc/ or include/."""
    if not obj.exists():
        return True
    deps = [src] + list(CSRC.glob("*.h")) + list((REPO / "include").glob("*.h"))
    return obj.stat().st_mtime < max(d.stat().st_mtime for d in deps)


def build(jobs: int = 8, only=None, incremental: bool = False) -> None:
    """Compile and link every library (incremental: only objects older than
    their source or a header are compiled again)."""
    BUILD.mkdir(exist_ok=True)
    for lib, srcs in LIBS.items():
        if only and lib not in only:
            continue
        objs = []
        todo = []
        for s in srcs:
            src = CSRC / s
            obj = BUILD / (s + ".o")
            objs.append(obj)
            if not incremental or _stale(src, obj):
                todo.append((src, obj))
        with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
            list(ex.map(lambda a: _compile(*a), todo))
        out = PKG / lib
        tmp = PKG / (lib + ".tmp")
        cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", str(tmp)] + [str(o) for o in objs]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError("link failed for {}".format(lib))
        os.replace(tmp, out)
    if not only or "_gefen_host" in only:
        build_host_ext()
    if not only or "test_helpers" in only:
        build_test_helpers()


def build_test_helpers() -> None:
    """HIP helpers that only the GPU tests load (tests/hip/*.hip -> lib*.so beside them)."""
    for src in sorted((REPO / "tests" / "hip").glob("*.hip")):
        out = src.with_name("lib" + src.stem + ".so")
        tmp = out.with_name(out.name + ".tmp")
        cmd = [HIPCC] + COMMON + ["-shared", str(src), "-o", str(tmp)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError("hipcc failed on {}".format(src.name))
        os.replace(tmp, out)


def build_host_ext() -> None:
    """_gefen_host: the host-side plan checks (csrc/host_plan.cpp), a CPython
    extension built with the host C++ compiler against torch's headers."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    torch_lib = cpp_extension.library_paths()[0]
    out = PKG / ("_gefen_host" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-shared", "-fPIC", "-std=c++17", "-Wall", "-ffp-contract=off",
           "-D_GLIBCXX_USE_CXX11_ABI={}".format(int(torch.compiled_with_cxx11_abi())),
           "-I", sysconfig.get_paths()["include"]]
    for inc in cpp_extension.include_paths():
        cmd += ["-I", inc]
    cmd += [str(CSRC / "host_plan.cpp"), "-o", str(tmp), "-L", torch_lib, "-Wl,-rpath," + torch_lib,
            "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("host extension build failed")
    os.replace(tmp, out)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--incremental", action="store_true",
                    help="compile only objects older than their source or a header")
    args = ap.parse_args()
    build(args.jobs, incremental=args.incremental)
    print("built", ", ".join(list(LIBS) + ["_gefen_host", "test helpers"]))
