"""The library's fp32 -> bf16 rounding (nanochat_amd/csrc/common.h: gfx950's v_cvt_pk_bf16_f32, packed and scalar)
equals the integer round-to-nearest-even rule with quiet NaNs for all 2^32 fp32 bit patterns, in both halves of the
packed instruction, built with the library's flags and with prefill_attn.hip's (no IEEE mode, no NaN semantics).
That rule is the oracle's bf16 rounding (oracle/golden.py), which the reference's __float2bfloat16_rn and torch's
.to(torch.bfloat16) follow for finite values. The probe (tests/gpu_probes/bf16_rounding.hip) is built in-tree by
__graft_entry__.build()."""

import ctypes
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

PROBES = Path(__file__).resolve().parent / "gpu_probes"


@pytest.mark.parametrize("name", ["libbf16_probe.so", "libbf16_probe_noieee.so"], ids=["ieee", "no-ieee"])
def test_hardware_bf16_rounding_equals_the_integer_rule_on_every_input(gpu, name):
    path = PROBES / name
    assert path.exists(), f"{path} is not built: run __graft_entry__.build()"
    print(f"bf16 rounding probe {name}: all 2^32 patterns", flush=True)
    lib = ctypes.CDLL(str(path))
    packed, scalar, first = ctypes.c_ulonglong(), ctypes.c_ulonglong(), ctypes.c_uint32()
    assert lib.bf16_probe(ctypes.byref(packed), ctypes.byref(scalar), ctypes.byref(first)) == 0
    assert packed.value == 0 and scalar.value == 0, (packed.value, scalar.value, hex(first.value))
