"""Build libaneforge_hip.so from aneforge_amd/csrc/*.hip with hipcc for gfx950.

The reference builds its native dispatch library with `xcrun clang++ -dynamiclib`
(aneforge/_lib/build.sh:8-11); this is the HIP equivalent.  Objects are compiled in
parallel into csrc/_build/ and linked in-tree, so the library travels with the source
tree to the GPU box.  Run `python -m aneforge_amd._build` or call build().

build(sanitize=True) makes the debug variant libaneforge_hip_asan.so: the host code of every
translation unit built with AddressSanitizer (the device code is not instrumented), linked by the
host compiler against the shared ASan runtime, which the loading process must preload
(asan_runtime() gives its path).  tests/test_asan_host.py drives the C ABI's host paths with it."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libaneforge_hip.so"
OUT_ASAN = PKG / "libaneforge_hip_asan.so"
ARCH = os.environ.get("AFX_OFFLOAD_ARCH", "gfx950")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
CLANGXX = os.path.join(ROCM, "llvm", "bin", "clang++")
# host-only instrumentation: -Xarch_host in front of each sanitizer flag keeps it off the device pass
ASAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer", "-g"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep hipcc from forming packed-fp32 VALU ops (v_pk_fma_f32 and friends)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    "-Wno-pass-failed",   # an occupancy target that LDS, not registers, already limits
    "-Werror=format",     # error messages are printf formats (set_error is declared as one)
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def asan_runtime() -> str:
    """Path of the compiler's shared AddressSanitizer runtime (LD_PRELOAD it to load the ASan build)."""
    r = subprocess.run([CLANGXX, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    return r.stdout.strip()


def build(verbose: bool = False, jobs: int | None = None, sanitize: bool = False) -> Path:
    """Compile every HIP source and link the shared library; returns its path.  sanitize=True builds
    the host-ASan variant (OUT_ASAN, objects in csrc/_build_asan)."""
    bdir = CSRC / ("_build_asan" if sanitize else "_build")
    out_path = OUT_ASAN if sanitize else OUT
    flags = CFLAGS + (ASAN_FLAGS if sanitize else [])
    bdir.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    procs: list[tuple[Path, subprocess.Popen]] = []
    objs = []
    pending = list(srcs)
    failed = []
    while pending or procs:
        while pending and len(procs) < jobs:
            s = pending.pop(0)
            o = bdir / (s.stem + ".o")
            objs.append(o)
            cmd = [HIPCC, *flags, "-I", str(CSRC), "-c", str(s), "-o", str(o)]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((s, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        s, p = procs.pop(0)
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        # the host pass does not know the packed-fp32 feature; that note is expected
        text = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            failed.append((s, text))
        elif verbose and text.strip():
            print(text, flush=True)
    if failed:
        msg = "\n".join(f"--- {s.name} ---\n{t}" for s, t in failed)
        raise RuntimeError(f"hipcc failed for {[s.name for s, _ in failed]}:\n{msg}")
    tmp = out_path.with_suffix(".so.tmp")
    if sanitize:   # a host link: the objects already carry their device code
        cmd = [CLANGXX, "-shared", "-fsanitize=address", "-shared-libasan", "-o", str(tmp), *map(str, objs),
               f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"]
    else:
        cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out_path)
    return out_path


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv, sanitize="--asan" in sys.argv)
    print(p)
