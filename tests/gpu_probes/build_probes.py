"""Builds the GPU probes that tests/test_gpu_bf16_rounding.py loads (test infrastructure, built in-tree by
__graft_entry__.build() like the library): bf16_rounding.hip twice, with the library's flags and with
prefill_attn.hip's additions (no IEEE mode, no NaN semantics)."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
if str(HERE.parents[1]) not in sys.path:
    sys.path.insert(0, str(HERE.parents[1]))

from nanochat_amd import build as lib_build  # noqa: E402
PROBES = {"libbf16_probe.so": [], "libbf16_probe_noieee.so": lib_build.FILE_FLAGS["prefill_attn.hip"]}


def build() -> None:
    src = HERE / "bf16_rounding.hip"
    for name, extra in PROBES.items():
        cmd = [lib_build.HIPCC, *lib_build.FLAGS, *extra, "-shared", str(src), "-o", str(HERE / name)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name} ({name}):\n{r.stderr}")
    print(f"built {len(PROBES)} GPU probes in {HERE}", file=sys.stderr)


if __name__ == "__main__":
    build()
