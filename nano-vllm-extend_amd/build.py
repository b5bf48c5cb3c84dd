"""Build recipe for libgdn_mi355x.so (gfx950).

Each csrc/*.hip translation unit is compiled with hipcc for gfx950 only; the
objects are linked with g++ against the HIP runtime that ships inside the
installed torch wheel (torch/lib/libamdhip64.so, soname libamdhip64.so.7) and
with no RUNPATH, so the library binds to the runtime torch has already
loaded instead of pulling a second copy from /opt/rocm.

Run as `python nano-vllm-extend_amd/build.py` or through
`__graft_entry__.build()`.  Output: nano-vllm-extend_amd/lib/libgdn_mi355x.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
OUT_DIR = PKG_DIR / "lib"
LIB_NAME = "libgdn_mi355x.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU ops are disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-file additions.  The chunk kernels read MFMA operands from LDS in long
# runs with one wave per SIMD; the ILP-oriented scheduler batches those reads
# ahead of their MFMAs instead of waiting on each pair in turn.
FILE_FLAGS = {
    "chunk_prefill.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the GDN extension)")


def _torch_lib_dir() -> Path:
    import torch  # noqa: F401  (only to locate its bundled HIP runtime)

    return Path(torch.__file__).resolve().parent / "lib"


def _compile(src: Path, obj: Path, extra: list[str]) -> tuple[Path, str]:
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns about the device-only target feature; drop that noise
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    return obj, msgs


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the C-ABI library."""
    extra = list(extra_flags or [])
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        futs = [ex.submit(_compile, s, obj_dir / (s.stem + ".o"), extra) for s in sources]
        objs = []
        for f in futs:
            obj, msgs = f.result()
            objs.append(obj)
            if verbose and msgs.strip():
                print(msgs, file=sys.stderr)
    tlib = _torch_lib_dir()
    out = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = ["g++", "-shared", "-o", str(tmp), *map(str, objs), f"-L{tlib}", "-lamdhip64",
           "-Wl,--no-undefined", "-Wl,-z,defs"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    p = build(verbose=True)
    print(p)
