"""The C-ABI library builds, loads and exports every entry point include/nanochat_amd.h declares, and its host-side
argument checks reject bad calls before any launch (CPU only: no compute call reaches a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

from nanochat_amd import native

HEADER = Path(__file__).resolve().parents[1] / "include" / "nanochat_amd.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^(?:[A-Za-z_]\w*\s+)+\**\s*(\w+)\s*\(", text, flags=re.M)


def test_header_declarations_match_the_bindings():
    names = declared_functions()
    assert len(names) >= 8
    assert set(names) == set(native.SIGNATURES), set(names) ^ set(native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = native.hip_library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.nc_abi_version() == 1


def test_workspace_query_is_pure_host():
    lib = native.hip_library()
    assert lib.nc_decode_workspace_bytes(0, 16, 4, 8192) == 0
    w = lib.nc_decode_workspace_bytes(64, 16, 4, 8193)
    assert w >= (8192 + 256) * 4 * 130 * 4  # a slot per wave and per segment, 4 heads of (128 + 2) floats
    assert lib.nc_decode_workspace_bytes(64, 16, 4, 100) == w  # the same for contexts up to about 8K keys


def test_workspace_follows_the_piece_cap():
    """The piece plan keeps up to max(32, ceil(ceil(max_ctx / 16) / 16)) pieces per (sequence, kv head), at most
    256, each with a slot of G (128 + 2) floats: past 8192 keys the workspace grows with max_ctx (once those slots
    outnumber the balanced split's), and from 65536 keys on it stays at 256 slots per segment."""
    lib = native.hip_library()
    slot = 4 * 130 * 4  # G = 4 heads of (128 + 2) floats
    ws = {c: lib.nc_decode_workspace_bytes(1024, 16, 4, c) for c in (4096, 8192, 32768, 65536, 131072, 1 << 20)}
    assert ws[4096] == ws[8192]
    assert ws[8192] < ws[32768] < ws[65536]
    assert ws[65536] == ws[131072] == ws[1 << 20]
    assert ws[65536] >= 4096 * 256 * slot  # 1024 x 4 segments of 256 slots
    assert ws[32768] >= 4096 * 128 * slot


NULL = ctypes.c_void_p(0)
FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails its host checks first


@pytest.mark.parametrize("kwargs, message", [
    (dict(hq=6, hkv=4), "multiple"),
    (dict(hq=64, hkv=2), "exceeds"),
    (dict(max_ctx=0), "max_ctx"),
    (dict(max_ctx=10_000), "max_ctx"),
    (dict(workspace_bytes=0), "workspace"),
    (dict(num_blocks=2), "contiguous"),
])
def test_decode_rejects_bad_arguments(kwargs, message):
    lib = native.hip_library()
    a = dict(hq=16, hkv=4, max_ctx=4096, workspace_bytes=1 << 30, num_blocks=1 << 16)
    a.update(kwargs)
    rc = lib.nc_decode_attn_fp8(FAKE, FAKE, NULL, 512, a["num_blocks"], FAKE, -1, 8, a["hq"], a["hkv"],
                                a["max_ctx"], 0.08, FAKE, FAKE, a["workspace_bytes"], NULL)
    assert rc < 0
    assert message in lib.nc_last_error().decode()


def test_decode_step_rejects_bad_arguments():
    lib = native.hip_library()
    qkv, out = 0x10000, 0x100000
    #       qkv                     row_stride pos   pos_out q_gain k_gain cos sin rope cache table max_b blocks
    base = [ctypes.c_void_p(qkv), 24 * 128, FAKE, NULL, FAKE, FAKE, FAKE, FAKE, 4096, FAKE, NULL, 512, 1 << 16,
            # window B hq  hkv max_ctx scale out                    workspace bytes    stream
            -1, 8, 16, 4, 4096, 0.08, ctypes.c_void_p(out), FAKE, 1 << 30, NULL]

    def rejects(i, value, message):
        args = list(base)
        args[i] = value
        assert lib.nc_decode_step_fp8(*args) < 0, (i, value)
        assert message in lib.nc_last_error().decode(), lib.nc_last_error()

    rejects(1, 100, "row_stride")
    rejects(15, 6, "multiple")
    rejects(15, 64 * 4, "row_stride")  # the row no longer holds the heads
    rejects(8, 0, "rope_len")
    rejects(4, NULL, "null")
    rejects(19, ctypes.c_void_p(qkv + 256), "overlap")
    rejects(3, FAKE, "pos_out")  # pos_out on pos
    rejects(17, 0, "max_ctx")
    rejects(21, 0, "workspace")
    rejects(12, 2, "contiguous")
    rejects(0, ctypes.c_void_p(qkv + 8), "aligned")
    empty = list(base)
    empty[14] = 0
    assert lib.nc_decode_step_fp8(*empty) == 0  # nothing to do, nothing launched


def test_append_rejects_bad_arguments():
    lib = native.hip_library()
    base = [FAKE, 1024, 4, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4096, 16, 4, FAKE, FAKE, NULL, 8, 64, 8, NULL, NULL]
    bad_stride = list(base)
    bad_stride[1] = 100
    assert lib.nc_kv_append_fp8(*bad_stride) < 0 and "row_stride" in lib.nc_last_error().decode()
    bad_heads = list(base)
    bad_heads[10] = 6
    assert lib.nc_kv_append_fp8(*bad_heads) < 0 and "multiple" in lib.nc_last_error().decode()
    null_cache = list(base)
    null_cache[13] = NULL
    assert lib.nc_kv_append_fp8(*null_cache) < 0 and "null" in lib.nc_last_error().decode()
    ctx_on_pos = list(base)
    ctx_on_pos[1] = (16 + 2 * 4) * 128
    ctx_on_pos[3] = ctx_on_pos[18] = ctypes.c_void_p(0x2000)  # ctx_out overlapping pos
    assert lib.nc_kv_append_fp8(*ctx_on_pos) < 0 and "overlap" in lib.nc_last_error().decode()
    assert lib.nc_kv_store_fp8(FAKE, FAKE, 100, 4, FAKE, FAKE, 4, FAKE, NULL, 8, 64, 8, NULL) < 0
    assert lib.nc_kv_gather_fp8(FAKE, NULL, 8, 64, FAKE, 8, 4, 200, FAKE, FAKE, FAKE, FAKE, NULL) < 0


def test_stale_library_is_detected(tmp_path, monkeypatch):
    from nanochat_amd import build

    assert build.is_current()
    monkeypatch.setattr(build, "STAMP", tmp_path / "missing.sha256")
    assert not build.is_current()


def test_prefill_rejects_bad_arguments():
    lib = native.hip_library()
    #       q     pos   seq   n   cache table max_blocks num_blocks num_seqs window hq hkv scale out   stream
    base = [FAKE, FAKE, FAKE, 64, FAKE, NULL, 8, 64, 8, -1, 16, 4, 0.08, FAKE, NULL]

    def rejects(i, value, message):
        args = list(base)
        args[i] = value
        assert lib.nc_prefill_attn_fp8(*args) < 0, (i, value)
        assert message in lib.nc_last_error().decode(), lib.nc_last_error()

    rejects(3, -1, "n = -1")
    rejects(10, 6, "hq % hkv")
    rejects(10, 68, "hq / hkv <= 16")
    rejects(7, 63, "contiguous")
    rejects(8, 0, "positive")
    rejects(4, NULL, "null")
    rejects(0, ctypes.c_void_p(0x1008), "aligned")
    empty = list(base)
    empty[3] = 0
    assert lib.nc_prefill_attn_fp8(*empty) == 0  # nothing to do, nothing launched


def test_argmax_rejects_bad_arguments():
    lib = native.hip_library()
    assert lib.nc_argmax_f32(FAKE, 4, 0, 10, FAKE, NULL) < 0 and "cols" in lib.nc_last_error().decode()
    assert lib.nc_argmax_f32(FAKE, 4, 10, 5, FAKE, NULL) < 0
    assert lib.nc_argmax_f32(NULL, 4, 10, 10, FAKE, NULL) < 0 and "null" in lib.nc_last_error().decode()
    assert lib.nc_argmax_f32(FAKE, 0, 10, 10, FAKE, NULL) == 0  # nothing to do, nothing launched


def test_slot_gemm_rejects_bad_arguments():
    lib = native.hip_library()

    def rejects(n, k, m, epi, res, tile, message):
        rc = lib.nc_slot_gemm_bf16(FAKE, n, k, FAKE, m, epi, FAKE, res, tile[0], tile[1], NULL)
        assert rc < 0
        assert message in lib.nc_last_error().decode(), lib.nc_last_error().decode()

    rejects(48, 64, 8, 0, NULL, (0, 0), "multiple of 32")
    rejects(32, 96, 8, 0, NULL, (0, 0), "multiple of 32")  # k % 64
    rejects(32, 64, 8, 5, NULL, (0, 0), "epilogue")
    rejects(32, 64, 8, 2, NULL, (0, 0), "RESID needs res")
    rejects(32, 64, 8, 0, NULL, (16, 16), "tile")
    rejects(32, 64, 8, 0, NULL, (48, 16), "tile")
    rejects(96, 64, 8, 0, NULL, (64, 32), "tile")  # n not a multiple of the tile
    rejects(1 << 20, 1 << 10, 8, 0, NULL, (0, 0), "2 GiB")
    assert lib.nc_slot_gemm_bf16(FAKE, 32, 64, FAKE, 0, 0, FAKE, NULL, 0, 0, NULL) == 0  # m = 0: nothing launched


def test_slot_gemm_prefetch_rejects_bad_arguments():
    """The prefetch range is checked before the GEMM's own arguments; the GEMM's checks still apply."""
    lib = native.hip_library()

    def rejects(pf, pf_bytes, n, message):
        rc = lib.nc_slot_gemm_bf16_prefetch(FAKE, n, 64, FAKE, 8, 0, FAKE, NULL, 0, 0, pf, pf_bytes, NULL)
        assert rc < 0
        assert message in lib.nc_last_error().decode(), lib.nc_last_error().decode()

    rejects(NULL, 65536, 32, "prefetch")       # bytes without a range
    rejects(FAKE, -1, 32, "prefetch")          # negative size
    rejects(ctypes.c_void_p(0x1008), 65536, 32, "prefetch")  # not 16-byte aligned
    rejects(FAKE, 65536, 48, "multiple of 32")  # a good range, a bad GEMM
    assert lib.nc_slot_gemm_bf16_prefetch(FAKE, 32, 64, FAKE, 0, 0, FAKE, NULL, 0, 0, FAKE, 65536, NULL) == 0  # m = 0


def test_choose_rejects_bad_arguments():
    lib = native.hip_library()
    need = lib.nc_choose_workspace_bytes(8, 1000)
    assert need >= 8 * 2 * 8  # a best and an alternative key per slot at least
    assert lib.nc_choose_workspace_bytes(0, 1000) == 0
    #       logits B  vocab ld   active allow temp  top_p seed  first pos   cap  lazy tokens alt  ws    bytes stream
    base = [FAKE, 8, 1000, 200_000, NULL, NULL, NULL, NULL, NULL, NULL, FAKE, 15.0, -1, FAKE, FAKE, FAKE, need, NULL]

    def rejects(i, value, message):
        args = list(base)
        args[i] = value
        assert lib.nc_choose_tokens(*args) < 0, (i, value)
        assert message in lib.nc_last_error().decode(), lib.nc_last_error()

    rejects(3, 999, "ld")
    rejects(2, 0, "vocab")
    rejects(2, 131073, "exceeds")
    rejects(10, NULL, "null")
    rejects(4, FAKE, "allow")           # a slot mask without the allowed-row masks
    rejects(6, FAKE, "seeds")           # temperatures without seeds
    rejects(16, need - 1, "workspace")
    rejects(15, ctypes.c_void_p(0x1008), "aligned")
    empty = list(base)
    empty[1] = 0
    assert lib.nc_choose_tokens(*empty) == 0


def test_value_embed_rejects_bad_arguments():
    lib = native.hip_library()
    #       qkv   stride x     xs   tok   ve    vocab gate  rows d    hq hkv stream
    base = [FAKE, 1024, FAKE, 256, FAKE, FAKE, 100, FAKE, 4, 256, 4, 2, NULL]

    def rejects(i, value, message):
        args = list(base)
        args[i] = value
        assert lib.nc_value_embed_bf16(*args) < 0, (i, value)
        assert message in lib.nc_last_error().decode(), lib.nc_last_error()

    rejects(9, 260, "d")            # not a multiple of 8
    rejects(9, 8200, "d")           # past the row limit
    rejects(11, 3, "hkv")           # does not divide hq
    rejects(11, 0, "hkv")
    rejects(1, 1016, "row_stride")  # narrower than hq + 2 hkv heads
    rejects(3, 248, "x_stride")
    rejects(6, 0, "vocab")
    rejects(4, NULL, "null")
    rejects(0, ctypes.c_void_p(0x1008), "alignment")
    empty = list(base)
    empty[8] = 0
    assert lib.nc_value_embed_bf16(*empty) == 0  # no rows, nothing launched


def test_decoder_handle_rejects_bad_configurations():
    """dec_create_v2 checks its configuration before any device call and returns NULL with a message."""
    import numpy as np

    lib = native.hip_library()
    ptrs = np.full(4 + 8 * 2, 0x1000, dtype=np.uint64)
    ptrs[4 + 4] = ptrs[4 + 5] = ptrs[12 + 4] = ptrs[12 + 5] = 0  # no value embeddings
    scal = np.array([1, 0, 1, 0, 15], dtype=np.float32)
    window = np.array([-1, -1], dtype=np.int32)

    def rejects(cfg, message):
        cfg = np.array(cfg, dtype=np.int32)
        h = lib.dec_create_v2(cfg.ctypes.data, len(cfg), ptrs.ctypes.data, scal.ctypes.data, window.ctypes.data, NULL)
        assert not h
        assert message in lib.nc_last_error().decode(), lib.nc_last_error()

    good = [2, 256, 1024, 1000, 48, 0, 7, 2, 4, 1]
    rejects(good[:6], "config fields")
    rejects([2, 200] + good[2:], "C 200")               # not a multiple of 128
    rejects(good[:2] + [1000] + good[3:], "F 1000")     # not a multiple of 64
    rejects(good[:3] + [200000] + good[4:], "vocab")
    rejects(good[:7] + [3] + good[8:], "kv heads")      # 2 heads over 3 kv heads
    rejects(good[:8] + [2000] + good[9:], "batch")      # more than 1024 slots
    bad = ptrs.copy()
    bad[4 + 8 + 1] = 0                                   # layer 1 without its o projection
    cfg = np.array(good, dtype=np.int32)
    assert not lib.dec_create_v2(cfg.ctypes.data, len(cfg), bad.ctypes.data, scal.ctypes.data, window.ctypes.data,
                                 NULL)
    assert "layer 1" in lib.nc_last_error().decode()


def test_embed_and_mix_reject_bad_arguments():
    lib = native.hip_library()
    assert lib.nc_embed_rms_norm(FAKE, 0, 100, FAKE, 4, 260, FAKE, NULL) < 0 and "d" in lib.nc_last_error().decode()
    assert lib.nc_embed_rms_norm(FAKE, 0, 0, FAKE, 4, 256, FAKE, NULL) < 0 and "vocab" in lib.nc_last_error().decode()
    assert lib.nc_embed_rms_norm(NULL, 0, 100, FAKE, 4, 256, FAKE, NULL) < 0
    assert lib.nc_embed_rms_norm(FAKE, 0, 100, FAKE, 0, 256, FAKE, NULL) == 0  # no rows, nothing launched
    assert lib.nc_mix_bf16(FAKE, FAKE, 12, 1.0, 0.0, NULL) < 0 and "multiple of 8" in lib.nc_last_error().decode()
    assert lib.nc_mix_bf16(NULL, FAKE, 16, 1.0, 0.0, NULL) < 0
    assert lib.nc_mix_bf16(FAKE, FAKE, 0, 1.0, 0.0, NULL) == 0


def test_a_c_caller_compiles_links_and_runs(tmp_path):
    """The header is plain C: a C program includes it, links libnanochat_amd.so and calls the host-only entry points
    (no device work), the way a C or cgo caller would."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    lib = Path(native.hip_library()._name)
    src = tmp_path / "caller.c"
    src.write_text('#include "nanochat_amd.h"\n#include <stdio.h>\n'
                   'int main(void) {\n'
                   '    printf("%d %lld %lld\\n", nc_abi_version(), nc_decode_workspace_bytes(64, 16, 4, 8192),\n'
                   '           nc_choose_workspace_bytes(8, 1000));\n'
                   '    return nc_decode_attn_fp8(0, 0, 0, 0, 0, 0, -1, 1, 16, 4, 16, 1.0f, 0, 0, 0, 0) < 0 ? 0 : 1;\n'
                   '}\n')
    exe = tmp_path / "caller"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{HEADER.parent}", str(src), f"-L{lib.parent}",
                    "-lnanochat_amd", f"-Wl,-rpath,{lib.parent}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out[0] == "1"
    assert int(out[1]) == native.hip_library().nc_decode_workspace_bytes(64, 16, 4, 8192)
    assert int(out[2]) == native.hip_library().nc_choose_workspace_bytes(8, 1000)


def test_reference_entry_dec_create_aborts_on_a_bad_configuration(tmp_path):
    """The reference's dec_create aborts with a message (decode.cu:927-931): its caller never checks the handle. A C
    program passes a hidden size that is not a multiple of 128; the check runs before any device call, so no GPU is
    needed, and the process ends by SIGABRT naming the problem."""
    import shutil
    import signal
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    lib = Path(native.hip_library()._name)
    src = tmp_path / "create.c"
    src.write_text('#include "nanochat_amd.h"\n#include <stdio.h>\n'
                   'int main(void) {\n'
                   '    int cfg[7] = {1, 200, 1024, 1000, 48, 0, 7};\n'
                   '    uint64_t ptrs[12] = {0};\n'
                   '    float scal[3] = {1, 0, 15};\n'
                   '    int window[1] = {-1};\n'
                   '    void *h = dec_create(cfg, ptrs, scal, window, 0);\n'
                   '    printf("returned %p\\n", h);\n'
                   '    return 0;\n'
                   '}\n')
    exe = tmp_path / "create"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{HEADER.parent}", str(src), f"-L{lib.parent}",
                    "-lnanochat_amd", f"-Wl,-rpath,{lib.parent}", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == -signal.SIGABRT, (r.returncode, r.stdout, r.stderr)
    assert "dec_create: " in r.stderr and "C 200" in r.stderr, r.stderr
    assert "returned" not in r.stdout


def test_position_rows_reject_bad_arguments():
    lib = native.hip_library()
    #          cache pool layers table max_b blocks seqs seq at n  hkv rows  stream
    base = [FAKE, 0, 1, NULL, 10, 40, 4, 1, 5, 20, 2, FAKE, NULL]

    def rejects(i, value, message):
        args = list(base)
        args[i] = value
        assert lib.nc_kv_export_fp8(*args) < 0, (i, value)
        assert message in lib.nc_last_error().decode(), lib.nc_last_error()

    rejects(7, 4, "sequence 4")         # past the 4 sequences
    rejects(8, 150, "positions")        # 150 + 20 > 10 pages of 16
    rejects(9, -1, "n -1")
    rejects(5, 30, "contiguous")        # 4 sequences x 10 blocks need 40
    rejects(2, 3, "pool_bytes")         # several layers need the pool stride
    rejects(0, NULL, "null")
    args = list(base)
    args[9] = 0
    assert lib.nc_kv_export_fp8(*args) == 0  # nothing to move: no launch
    # import takes the same checks (rows first, then the cache arguments)
    assert lib.nc_kv_import_fp8(FAKE, 1, FAKE, 0, NULL, 10, 40, 4, 9, 0, 3, 2, NULL) < 0
    assert "sequence 9" in lib.nc_last_error().decode()
