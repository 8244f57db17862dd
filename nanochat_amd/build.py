"""Build recipe of the HIP library: every csrc/*.hip compiled by hipcc for gfx950 into one in-tree shared object,
libnanochat_amd.so, loaded with ctypes (the reference builds each model/kernels/<name>.cu with nvcc the same way,
native.py:54-65).

The library sits next to this file with a sidecar `<lib>.sha256` holding the digest of the command and every
source and header, so a stale library is detected at load time (native.hip_library) and rebuilt.
"""

from __future__ import annotations

import hashlib
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIBRARY = PACKAGE / "libnanochat_amd.so"
STAMP = LIBRARY.with_suffix(".so.sha256")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 anywhere (hipcc would otherwise form them from float2 code).
# -amdgpu-mfma-vgpr-form: MFMA accumulators in VGPRs, so the softmax rescales of the decode kernel's output
# accumulators need no AGPR <-> VGPR copies.
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wshadow", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form",
         f"-I{PACKAGE.parent / 'include'}"]

# Per-source additions. prefill_attn.hip: no IEEE mode and no NaN semantics, so fmaxf compiles to plain v_max
# without NaN-quieting canonicalisations (the kernel's inputs are finite; a NaN in q or the cache has no meaning).
FILE_FLAGS = {"prefill_attn.hip": ["-mno-amdgpu-ieee", "-fno-honor-nans"]}


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def digest() -> str:
    """Of the command (with the repository-relative include path, so a copy of the tree elsewhere, e.g. on the GPU
    box, sees the same digest) and of every source and header."""
    flags = [f.replace(str(PACKAGE.parent), ".") for f in FLAGS]
    h = hashlib.sha256(" ".join([os.path.basename(HIPCC), *flags, repr(sorted(FILE_FLAGS.items()))]).encode())
    for f in sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.h"), *(PACKAGE.parent / "include").glob("*.h")]):
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()


def is_current() -> bool:
    return LIBRARY.exists() and STAMP.exists() and STAMP.read_text().strip() == digest()


def build(verbose: bool = True) -> Path:
    """Compile every source (in parallel) and link; the library is replaced atomically."""
    srcs = sources()
    stamp = digest()
    with tempfile.TemporaryDirectory(dir=PACKAGE) as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in srcs]

        def compile_one(pair):
            src, obj = pair
            cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
            if verbose and r.stderr.strip():
                filtered = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln]
                if filtered:
                    print("\n".join(filtered), file=sys.stderr)
            return obj

        with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
            list(pool.map(compile_one, zip(srcs, objs)))
        out = Path(tmp) / LIBRARY.name
        r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(out), *map(str, objs)],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr}")
        out.replace(LIBRARY)
    STAMP.write_text(stamp + "\n")
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build()
