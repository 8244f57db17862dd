"""Pins of the CPU oracle (oracle/golden.py) against library routines, closed forms and brute force. CPU only.

Each check is chosen so that a plausible slip in the oracle (a dropped term, a wrong sign or index, a transposed
operand, a wrong rounding mode) fails it; none retypes the oracle's own formula."""

import math

import numpy as np
import torch

from oracle import golden as G


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ----------------------------------------------------------------------------------------------- rounding primitives

def special_floats() -> np.ndarray:
    vals = [0.0, -0.0, 1.0, -1.0, 448.0, -448.0, 463.99, 464.0, 464.00003, 470.0, 480.0, 1e6, np.inf, -np.inf,
            2.0 ** -6, 2.0 ** -7, 2.0 ** -9, 2.0 ** -10, 1.5 * 2.0 ** -10, 3 * 2.0 ** -11, 2.0 ** -6 * (1 - 2 ** -24),
            2.0 ** -100, 1e-40]
    grid = np.array(vals, np.float32)
    # every fp32 tie and near-tie around each e4m3 code
    codes = G.E4M3_TABLE[np.isfinite(G.E4M3_TABLE)]
    mids = ((codes[:-1].astype(np.float64) + codes[1:]) / 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    return np.concatenate([grid, -grid, codes, mids, near])


def test_e4m3_encode_matches_torch_cast():
    """Library pin: torch's float32 -> float8_e4m3fn cast (RNE, NaN beyond 464) on specials, every tie between
    adjacent codes and 2M random bit patterns of all magnitudes."""
    rng = np.random.default_rng(0)
    rand = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rand = rand[np.isfinite(rand)]
    scaled = (rng.standard_normal(1_000_000) * 100).astype(np.float32)
    for x in (special_floats(), rand, scaled):
        want = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        got = G.e4m3_encode(x)
        nan_want = (want & 0x7F) == 0x7F
        np.testing.assert_array_equal(nan_want, (got & 0x7F) == 0x7F)
        np.testing.assert_array_equal(got[~nan_want], want[~nan_want])


def test_e4m3_decode_matches_torch_exhaustively():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = G.e4m3_decode(codes)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
    # the format's fixed points: max 448, smallest normal 2^-6, smallest subnormal 2^-9
    assert G.E4M3_TABLE[0x7E] == 448 and G.E4M3_TABLE[0x08] == 2 ** -6 and G.E4M3_TABLE[0x01] == 2 ** -9


def test_e4m3_round_trip_all_codes():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
    np.testing.assert_array_equal(G.e4m3_encode(G.e4m3_decode(codes)), codes)


def test_bf16_bits_matches_torch_cast():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.integers(0, 2 ** 32, 1_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                        special_floats()])
    x = x[~np.isnan(x)]
    want = bits_of(torch.from_numpy(x.copy()).to(torch.bfloat16))
    np.testing.assert_array_equal(G.bf16_bits(x), want)
    np.testing.assert_array_equal(G.bf16_to_f32(want), torch.from_numpy(want.view(np.int16)).view(
        torch.bfloat16).float().numpy())


# ----------------------------------------------------------------------------------------------- rotary + row math

def test_rotary_tables_closed_form():
    theta = 10000.0
    cos, sin = G.rotary_tables(4096, theta)
    assert cos.dtype == np.float32 and cos.shape == (4096, 64)
    np.testing.assert_array_equal(cos[0], 1.0)
    np.testing.assert_array_equal(sin[0], 0.0)
    for t, i in [(1, 0), (1, 63), (4095, 0), (4095, 17), (2048, 63), (37, 5)]:
        ang = t * theta ** (-2 * i / 128)
        assert cos[t, i] == np.float32(math.cos(ang)) and sin[t, i] == np.float32(math.sin(ang))
    # frequency 0 rotates by exactly t radians
    t = np.arange(4096)
    np.testing.assert_array_equal(cos[:, 0], np.cos(t.astype(np.float64)).astype(np.float32))


def test_sum_squares_accuracy_and_exact_cases():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1000, 128)).astype(np.float32)
    exact = (x.astype(np.float64) ** 2).sum(-1)
    got = G.sum_squares(x).astype(np.float64)
    assert np.all(np.abs(got - exact) <= exact * 9 * 2.0 ** -24)  # tree depth 8 + product rounding
    np.testing.assert_array_equal(G.sum_squares(np.full((3, 128), 0.5, np.float32)), np.float32(32.0))
    one_hot = np.zeros((128, 128), np.float32)
    one_hot[np.arange(128), np.arange(128)] = 3.0
    np.testing.assert_array_equal(G.sum_squares(one_hot), np.float32(9.0))


def bf16_ulp(y: np.ndarray) -> np.ndarray:
    e = np.floor(np.log2(np.maximum(np.abs(y), 1e-30)))
    return 2.0 ** (e - 7)


def random_bf16(shape, seed, scale=1.0) -> np.ndarray:
    g = torch.Generator().manual_seed(seed)
    return bits_of((torch.randn(shape, generator=g) * scale).to(torch.bfloat16))


def test_qk_norm_rope_identity_rotation_is_rms_norm():
    """pos 0 (cos 1, sin 0), gain 1: y = x / sqrt(mean x² + eps), within one bf16 rounding of the fp64 value."""
    x = random_bf16((64, 128), 3, scale=3.0)
    y = G.bf16_to_f32(G.qk_norm_rope(x, np.ones(128, np.float32), np.ones(64, np.float32),
                                     np.zeros(64, np.float32))).astype(np.float64)
    xf = G.bf16_to_f32(x).astype(np.float64)
    want = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + float(G.EPS))
    assert np.all(np.abs(y - want) <= bf16_ulp(want) * 0.5 + np.abs(want) * 2.0 ** -20)


def test_qk_norm_rope_one_hot_rstd():
    """x = c e_j: r = 1 / sqrt(c²/128 + eps) so y_j = c r exactly rounded; other dims 0."""
    for j in (0, 5, 63, 64, 127):
        x = np.zeros(128, np.float32)
        x[j] = 2.0
        y = G.bf16_to_f32(G.qk_norm_rope(G.bf16_bits(x), np.ones(128, np.float32), np.ones(64, np.float32),
                                         np.zeros(64, np.float32)))
        want = 2.0 / math.sqrt(4.0 / 128 + float(G.EPS))
        assert abs(y[j] - want) <= bf16_ulp(np.array(want)) / 2
        assert np.count_nonzero(y) == 1


def test_qk_norm_rope_pure_pair_rotates_by_minus_theta():
    """A row holding only the pair (i, i+64) rotates in that plane by -t θ^(-2i/128) (rotation by -θ, qk_row.cuh:3)
    with its length kept; the gain scales the normed value per dim before the rotation."""
    cos, sin = G.rotary_tables(512, 10000.0)
    for t, i in [(1, 0), (7, 3), (300, 40), (511, 63)]:
        x = np.zeros(128, np.float32)
        x[i], x[i + 64] = 1.0, 0.5
        g = np.ones(128, np.float32)
        g[i + 64] = 2.0  # n = (r, 2 * 0.5 r): the gained pair is (r, r)
        y = G.bf16_to_f32(G.qk_norm_rope(G.bf16_bits(x), g, cos[t], sin[t])).astype(np.float64)
        r = 1 / math.sqrt((1 + 0.25) / 128 + float(G.EPS))
        ang = t * 10000.0 ** (-2 * i / 128)
        want1 = r * math.cos(ang) + r * math.sin(ang)
        want2 = r * math.cos(ang) - r * math.sin(ang)
        assert abs(y[i] - want1) <= bf16_ulp(np.array(want1)) + 1e-5
        assert abs(y[i + 64] - want2) <= bf16_ulp(np.array(want2)) + 1e-5
        assert np.count_nonzero(y) <= 2


def test_qk_norm_rope_preserves_norm_and_is_row_local():
    cos, sin = G.rotary_tables(64, 1e6)
    x = random_bf16((8, 6, 128), 4)
    pos = np.arange(8) * 7
    y = G.qk_norm_rope(x, np.ones(128, np.float32), cos[pos][:, None], sin[pos][:, None])
    yf = G.bf16_to_f32(y).astype(np.float64)
    np.testing.assert_allclose(np.sqrt((yf ** 2).mean(-1)), 1.0, rtol=4e-3)
    # row locality: one row alone gives the same bits as within the batch
    np.testing.assert_array_equal(G.qk_norm_rope(x[3, 2], np.ones(128, np.float32), cos[pos[3]], sin[pos[3]]),
                                  y[3, 2])


# ----------------------------------------------------------------------------------------------- quantisation

def test_quantize_rows_known_answers():
    rng = np.random.default_rng(5)
    # absmax 448 * 2^k: the scale is exactly 2^k and codes are the plain e4m3 rounding of x / 2^k
    for k in (-3, 0, 2):
        x = (rng.uniform(-448, 448, (4, 128)) * 2.0 ** k).astype(np.float32)
        x[:, 7] = 448 * 2.0 ** k
        xb = G.bf16_bits(x)
        codes, scale = G.quantize_rows(xb)
        np.testing.assert_array_equal(scale, np.float32(2.0 ** k))
        want = torch.from_numpy(G.bf16_to_f32(xb) / np.float32(2.0 ** k)).to(torch.float8_e4m3fn).view(
            torch.uint8).numpy()
        np.testing.assert_array_equal(codes, want)
    # zero row: scale 0, codes 0, dequantises to 0
    codes, scale = G.quantize_rows(np.zeros((2, 128), np.uint16))
    assert np.all(codes == 0) and np.all(scale == 0)
    assert np.all(G.dequantize(codes, scale) == 0)


def test_quantize_rows_absmax_maps_to_448_and_error_bound():
    x = random_bf16((512, 128), 6)
    x[::7, 3] = G.bf16_bits(np.float32(-8.0))  # outliers move only the scale
    codes, scale = G.quantize_rows(x)
    xf = G.bf16_to_f32(x)
    amax = np.abs(xf).argmax(-1)
    np.testing.assert_array_equal(codes[np.arange(512), amax] & 0x7F, 0x7E)
    xq = G.dequantize(codes, scale)
    # half an e4m3 step: 2^-4 relative for normals (plus the dequantise rounding), 2^-10 scale below 2^-6 scale
    bound = np.maximum(np.abs(xf) * (2.0 ** -4 + 2.0 ** -23), scale[:, None] * 2.0 ** -10) * (1 + 1e-6)
    assert np.all(np.abs(xq - xf) <= bound)
    assert not np.any(np.isnan(xq))


# ----------------------------------------------------------------------------------------------- cache layout

def test_cache_layout_byte_offsets():
    """Tile (block, head) at byte (block * Hkv + head) * 4224 of the pool; K key 13, V key 13 at hand-computed bytes
    (K dims 0 / 20 / 77 / 127 at 208 / 1236 / 733 / 2015, V dims 0 / 5 / 77 / 127 at 2049 + 16 * 48 = 2817,
    3073 + 16 * 48 + 4, 3073 + 16 * 57 + 4, 3073 + 16 * 63 + 12), K scale t at 4096 + 4t, V scale t at
    4160 + 4t."""
    c = G.PagedCache(3, 2)
    kc = np.arange(128, dtype=np.uint8)
    vc = (np.arange(128) + 100).astype(np.uint8)
    c.write(np.array([2]), 1, np.array([13]), kc[None], np.float32(0.5), vc[None], np.float32(0.25))
    flat = c.pages.reshape(-1)
    tile = (2 * 2 + 1) * 4224
    for d, at in ((0, 208), (20, 1024 + 13 * 16 + 4), (77, (13 + 32) * 16 + 13), (127, 1024 + (13 + 48) * 16 + 15)):
        assert flat[tile + at] == kc[d], d
    for d, at in ((0, 2048 + 48 * 16 + 1), (5, 3072 + 48 * 16 + 4 + 1), (77, 3072 + (9 + 48) * 16 + 4 + 1),
                  (127, 3072 + (15 + 48) * 16 + 12 + 1)):
        assert flat[tile + at] == vc[d], d
    assert flat[tile + 4096 + 4 * 13: tile + 4096 + 4 * 14].view(np.float32)[0] == 0.5
    assert flat[tile + 4160 + 4 * 13: tile + 4160 + 4 * 14].view(np.float32)[0] == 0.25
    # 127 nonzero K codes, 128 V codes, and the scales' nonzero bytes: 0.5 = 0x3f000000 (1), 0.25 = 0x3e800000 (2)
    assert np.count_nonzero(flat) == 127 + 128 + 1 + 2


def test_host_byte_tables_match_the_layout():
    """nanochat_amd.kv_cache's K_BYTES / V_BYTES (what host code indexes the device pool with) are the oracle's, and
    the two tables cover a tile's 4096 code bytes once each."""
    from nanochat_amd.kv_cache import K_BYTES, V_BYTES
    np.testing.assert_array_equal(K_BYTES.numpy(), G.K_BYTES)
    np.testing.assert_array_equal(V_BYTES.numpy(), G.V_BYTES)
    both = np.concatenate([G.K_BYTES.ravel(), G.V_BYTES.ravel()])
    np.testing.assert_array_equal(np.sort(both), np.arange(4096))


def test_cache_parts_are_the_lanes_mfma_fragments():
    """Each 1 KiB part of a tile, read as [64 lanes][16 B], is what lane f = n + 16 j holds for the MFMAs: K part P,
    key n, dims 32 j + 16 P .. + 15 (16x16x32 A operand: row n, k slots of group j); V part 2 + P, dims
    8 n + 4 P .. 8 n + 4 P + 3 of keys 4 j .. 4 j + 3, one dword per dim with key 4 j + i in byte i."""
    c = G.PagedCache(1, 1)
    t = np.arange(16)
    dims = np.broadcast_to(np.arange(128, dtype=np.uint8), (16, 128))
    keys = np.broadcast_to((np.arange(16, dtype=np.uint8) + 128)[:, None], (16, 128))
    c.write(np.zeros(16, np.int64), 0, t, dims, np.float32(1), keys, np.float32(1))  # K code = dim, V code = key
    tile = c.pages[0, 0]
    for f in range(64):
        n, j = f % 16, f // 16
        for P in range(2):
            frag = tile[P * 1024 + 16 * f: P * 1024 + 16 * f + 16]
            np.testing.assert_array_equal(frag, 32 * j + 16 * P + np.arange(16))  # key n's dims: K codes are dims
            vfrag = tile[2048 + P * 1024 + 16 * f: 2048 + P * 1024 + 16 * f + 16].reshape(4, 4)  # [dim][key]
            np.testing.assert_array_equal(vfrag, np.broadcast_to(128 + 4 * j + np.arange(4), (4, 4)))
    # V dims: plant one code per (key, dim) and read the dword layout back
    rng = np.random.default_rng(3)
    vcodes = rng.integers(0, 256, (16, 128), dtype=np.uint8)
    c.write(np.zeros(16, np.int64), 0, t, dims, np.float32(1), vcodes, np.float32(1))
    tile = c.pages[0, 0]
    for f in (0, 5, 17, 40, 63):
        n, j = f % 16, f // 16
        for P in range(2):
            vfrag = tile[2048 + P * 1024 + 16 * f: 2048 + P * 1024 + 16 * f + 16].reshape(4, 4)
            np.testing.assert_array_equal(vfrag, vcodes[4 * j: 4 * j + 4, 8 * n + 4 * P: 8 * n + 4 * P + 4].T)


def test_append_then_gather_paged_equals_contiguous():
    """A random page permutation stores the same rows as the contiguous layout (brute-force comparison)."""
    hq, hkv, n_seq, max_blocks = 4, 2, 3, 4
    cos, sin = G.rotary_tables(64, 10000.0)
    rng = np.random.default_rng(7)
    pos = np.concatenate([np.arange(L) for L in (17, 64, 5)])
    seq = np.concatenate([np.full(L, b) for b, L in enumerate((17, 64, 5))])
    qkv = random_bf16((len(pos), (hq + 2 * hkv) * 128), 8)
    gq, gk = rng.uniform(0.5, 1.5, 128).astype(np.float32), rng.uniform(0.5, 1.5, 128).astype(np.float32)
    contig = G.PagedCache(n_seq * max_blocks, hkv)
    q1 = G.append(contig, qkv, pos, seq, gq, gk, cos, sin, hq, hkv, None, max_blocks)
    table = rng.permutation(n_seq * max_blocks).reshape(n_seq, max_blocks).astype(np.int32)
    paged = G.PagedCache(n_seq * max_blocks, hkv)
    q2 = G.append(paged, qkv, pos, seq, gq, gk, cos, sin, hq, hkv, table, max_blocks)
    np.testing.assert_array_equal(q1, q2)
    ctx = np.array([17, 64, 5])
    a = G.gather(contig, None, max_blocks, ctx, 64)
    b = G.gather(paged, table, max_blocks, ctx, 64)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    # the gathered rows are the directly quantised rows (q/k norm+rope'd at their positions, v as is)
    heads = qkv.reshape(len(pos), hq + 2 * hkv, 128)
    k_bits = G.qk_norm_rope(heads[:, hq:hq + hkv], gk, cos[pos][:, None], sin[pos][:, None])
    kc, ks = G.quantize_rows(k_bits)
    vc, vs = G.quantize_rows(heads[:, hq + hkv:])
    i = 17 + 9  # sequence 1, position 9
    np.testing.assert_array_equal(a[0][1, :, 9], kc[i])
    np.testing.assert_array_equal(a[1][1, :, 9], vc[i])
    np.testing.assert_array_equal(a[2][1, :, 9], ks[i])
    np.testing.assert_array_equal(a[3][1, :, 9], vs[i])
    # untouched positions stay zero
    assert np.all(a[0][2, :, 5:] == 0)


def test_export_rows_reads_the_tile_bytes_and_matches_gather():
    """A position's row is its K codes, V codes (dim order) and the two scales' bytes, read from the tile offsets of
    the layout formula (planted in the raw pool, not through the oracle's views), for any start and length; rows of
    a paged sequence equal gather's canonical rows at the same positions; a missing block gives a zero row."""
    hkv, max_blocks = 2, 5
    c = G.PagedCache(12, hkv)
    rng = np.random.default_rng(11)
    c.pages[...] = rng.integers(0, 256, c.pages.shape, dtype=np.uint8)
    table = np.array([[7, 3, 11, 0, -1], [1, 2, 4, 5, 6]], np.int32)
    flat = c.pages.reshape(-1)
    pos, h = 37, 1  # sequence 0, page 2 (block 11), token 5
    tile = (11 * hkv + h) * 4224
    rows = G.export_rows(c, table, max_blocks, 0, 30, 20)  # positions 30..49, unaligned both ends
    row = rows[pos - 30, h]
    kd = [(d // 16 % 2) * 1024 + (5 + 16 * (d // 32)) * 16 + d % 16 for d in range(128)]  # key 5 of the tile
    vd = [2048 + (d // 4 % 2) * 1024 + (d // 8 + 16 * (5 // 4)) * 16 + d % 4 * 4 + 5 % 4 for d in range(128)]
    np.testing.assert_array_equal(row[:128], flat[tile + np.array(kd)])
    np.testing.assert_array_equal(row[128:256], flat[tile + np.array(vd)])
    np.testing.assert_array_equal(row[256:260], flat[tile + 4096 + 20: tile + 4096 + 24])
    np.testing.assert_array_equal(row[260:264], flat[tile + 4160 + 20: tile + 4160 + 24])
    k, v, ks, vs = G.gather(c, table, max_blocks, np.array([64, 64]), 64)
    for i in range(20):
        if (30 + i) // 16 == 4:  # the missing block
            assert not rows[i].any()
            continue
        for hh in range(hkv):
            np.testing.assert_array_equal(rows[i, hh, :128], k[0, hh, 30 + i])
            np.testing.assert_array_equal(rows[i, hh, 128:256], v[0, hh, 30 + i])
            np.testing.assert_array_equal(rows[i, hh, 256:].view(np.float32), [ks[0, hh, 30 + i], vs[0, hh, 30 + i]])


def test_import_rows_moves_positions_and_nothing_else():
    """Rows exported from one sequence and imported at another start of another sequence land exactly there (the
    moved positions gather equal), every other byte of the pool is unchanged, and a missing block is not written."""
    hkv, max_blocks = 3, 4
    src = G.PagedCache(8, hkv)
    rng = np.random.default_rng(12)
    src.pages[...] = rng.integers(0, 256, src.pages.shape, dtype=np.uint8)
    rows = G.export_rows(src, None, max_blocks, 1, 3, 29)  # sequence 1 (blocks 4..7), positions 3..31
    dst = G.PagedCache(8, hkv)
    dst.pages[...] = rng.integers(0, 256, dst.pages.shape, dtype=np.uint8)
    before = dst.pages.copy()
    table = np.array([[2, 0, 6, -1], [1, 3, 4, 5]], np.int32)
    G.import_rows(dst, rows, table, max_blocks, 0, 21)  # positions 21..49 of sequence 0: blocks 0, 6, then missing
    a = G.gather(src, None, max_blocks, np.array([0, 32]), 32)
    b = G.gather(dst, table, max_blocks, np.array([48, 0]), 48)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x[1, :, 3:30], y[0, :, 21:48])
    changed = np.flatnonzero((dst.pages != before).any(axis=(1, 2)))
    assert set(changed) <= {0, 6}, changed  # only the blocks of pages 1 and 2 of sequence 0
    untouched = G.export_rows(dst, table, max_blocks, 0, 0, 21)  # positions before `at` keep their bytes
    np.testing.assert_array_equal(untouched, G.export_rows(_with(before, hkv), table, max_blocks, 0, 0, 21))


def _with(pages, hkv):
    c = G.PagedCache(pages.shape[0], hkv)
    c.pages[...] = pages
    return c


# ----------------------------------------------------------------------------------------------- attention

def make_cache(ctx, hkv, seed, table=False):
    max_blocks = -(-max(ctx) // G.PAGE)
    c = G.PagedCache(len(ctx) * max_blocks, hkv)
    rng = np.random.default_rng(seed)
    bt = rng.permutation(len(ctx) * max_blocks).reshape(len(ctx), max_blocks).astype(np.int32) if table else None
    for b, L in enumerate(ctx):
        t = np.arange(L)
        blk = G.PagedCache.block_of(np.full(L, b), t, bt, max_blocks)
        for h in range(hkv):
            kc, ks = G.quantize_rows(random_bf16((L, 128), seed * 100 + b * 10 + h))
            vc, vs = G.quantize_rows(random_bf16((L, 128), seed * 100 + b * 10 + h + 5))
            c.write(blk, h, t % G.PAGE, kc, ks, vc, vs)
    return c, bt, max_blocks


def test_decode_attention_special_cases():
    hq, hkv = 4, 2
    scale = 128 ** -0.5
    c, bt, mb = make_cache([1, 40, 40], hkv, 9)
    q = random_bf16((3, hq, 128), 10)
    out = G.decode_attention(q, c, bt, mb, np.array([1, 40, 40]), -1, hq, hkv, scale)
    k, v, ks, vs = G.gather(c, bt, mb, np.array([1, 40, 40]), 40)
    # one key: the output is that key's dequantised value, for every query head of the kv head
    for h in range(hq):
        np.testing.assert_allclose(out[0, h], G.dequantize(v[0, h // 2, 0], vs[0, h // 2, 0]), rtol=1e-12)
    # q = 0: uniform weights, the mean of V over the window
    q0 = np.zeros_like(q)
    out0 = G.decode_attention(q0, c, bt, mb, np.array([1, 40, 40]), 9, hq, hkv, scale)
    want = G.dequantize(v[1, 0, 30:40], vs[1, 0, 30:40]).astype(np.float64).mean(0)
    np.testing.assert_allclose(out0[1, 0], want, rtol=1e-12, atol=1e-15)
    # window >= context is full attention
    full = G.decode_attention(q, c, bt, mb, np.array([1, 40, 40]), 39, hq, hkv, scale)
    np.testing.assert_array_equal(full, out)


def test_decode_attention_brute_force_and_gqa_mapping():
    """Per-key Python loop (exp / sum), and GQA equals MHA over kv heads repeated G times."""
    hq, hkv = 6, 2
    scale = 0.1
    ctx = np.array([23, 7])
    c, bt, mb = make_cache(list(ctx), hkv, 11, table=True)
    q = random_bf16((2, hq, 128), 12)
    out = G.decode_attention(q, c, bt, mb, ctx, 5, hq, hkv, scale)
    k, v, ks, vs = G.gather(c, bt, mb, ctx, 23)
    qf = G.bf16_to_f32(q).astype(np.float64)
    for b in range(2):
        p = int(ctx[b]) - 1
        for h in range(hq):
            kh = h // 3
            keys = range(max(p - 5, 0), p + 1)
            w = [math.exp(float(qf[b, h] @ G.dequantize(k[b, kh, j], ks[b, kh, j]).astype(np.float64)) * scale)
                 for j in keys]
            acc = sum(wj * G.dequantize(v[b, kh, j], vs[b, kh, j]).astype(np.float64) for wj, j in zip(w, keys))
            np.testing.assert_allclose(out[b, h], acc / sum(w), rtol=1e-10, atol=1e-12)
    # MHA copy: kv head h of the 6-head cache is kv head h // 3 of the 2-head one
    mha = G.PagedCache(c.num_blocks, hq)
    for h in range(hq):
        mha.pages[:, h] = c.pages[:, h // 3]
    np.testing.assert_allclose(G.decode_attention(q, mha, bt, mb, ctx, 5, hq, hq, scale), out, rtol=1e-13)


def test_prefill_attention_reduces_to_decode_and_is_causal():
    hq, hkv = 4, 1
    scale = 128 ** -0.5
    ctx = [48, 33]
    c, bt, mb = make_cache(ctx, hkv, 13, table=True)
    q = random_bf16((16 + 5, hq, 128), 14)
    cu = np.array([0, 16, 21])
    start = np.array([32, 28])  # chunk rows are the sequences' last positions
    out = G.prefill_attention(q, cu, start, c, bt, mb, -1, hq, hkv, scale)
    for b, (r0, r1) in enumerate([(0, 16), (16, 21)]):
        for i in range(r1 - r0):
            # a batch of the one sequence b: its own block-table row
            d = G.decode_attention(q[r0 + i][None], c, bt[b:b + 1], mb, np.array([start[b] + i + 1]), -1, hq, hkv,
                                   scale)
            np.testing.assert_allclose(out[r0 + i], d[0], rtol=1e-12)
    # causality: changing keys after a row's position leaves that row unchanged
    c.pages[bt[0, 2], 0, G.K_BYTES[15]] ^= 0x11  # position 47 of sequence 0
    out2 = G.prefill_attention(q, cu, start, c, bt, mb, -1, hq, hkv, scale)
    np.testing.assert_array_equal(out2[:15], out[:15])
    assert not np.array_equal(out2[15], out[15])


def test_rows_attention_matches_chunks_any_order_and_skips_invalid_rows():
    """The per-row restatement equals the per-chunk one, is equivariant under any row order, gives zero rows for
    invalid (pos, seq) and with a window keeps only the last window + 1 keys."""
    hq, hkv = 6, 2
    scale = 128 ** -0.5
    ctx = [70, 45]
    c, bt, mb = make_cache(ctx, hkv, 21, table=True)
    q = random_bf16((30 + 12, hq, 128), 22)
    cu, start = np.array([0, 30, 42]), np.array([40, 33])
    pos = np.concatenate([start[0] + np.arange(30), start[1] + np.arange(12)])
    seq = np.repeat([0, 1], [30, 12])
    for window in (-1, 7):
        want = G.prefill_attention(q, cu, start, c, bt, mb, window, hq, hkv, scale)
        got = G.rows_attention(q, pos, seq, c, bt, mb, 2, window, hq, hkv, scale)
        np.testing.assert_array_equal(got, want)
        perm = np.random.default_rng(23).permutation(len(pos))
        shuffled = G.rows_attention(q[perm], pos[perm], seq[perm], c, bt, mb, 2, window, hq, hkv, scale)
        np.testing.assert_allclose(shuffled, want[perm], rtol=1e-13, atol=1e-15)
    bad_pos, bad_seq = pos.copy(), seq.copy()
    bad_pos[3], bad_seq[5], bad_seq[6] = -1, 2, -4
    out = G.rows_attention(q, bad_pos, bad_seq, c, bt, mb, 2, -1, hq, hkv, scale)
    assert not out[[3, 5, 6]].any()
    keep = np.setdiff1d(np.arange(len(pos)), [3, 5, 6])
    np.testing.assert_array_equal(out[keep], G.rows_attention(q, pos, seq, c, bt, mb, 2, -1, hq, hkv, scale)[keep])


def test_missing_blocks_are_skipped():
    """A hole in the block table removes that page's keys: the same as attending the remaining keys directly;
    a row whose keys are all missing is zero."""
    hq, hkv = 2, 1
    scale = 128 ** -0.5
    c, bt, mb = make_cache([64], hkv, 31, table=True)
    q = random_bf16((1, hq, 128), 32)
    holed = bt.copy()
    holed[0, 1] = -1  # keys 16..31
    out = G.decode_attention(q, c, holed, mb, np.array([64]), -1, hq, hkv, scale)
    k, v, ks, vs = G.gather(c, bt, mb, np.array([64]), 64)
    keep = np.r_[0:16, 32:64]
    kd = G.dequantize(k[0, 0, keep], ks[0, 0, keep]).astype(np.float64)
    vd = G.dequantize(v[0, 0, keep], vs[0, 0, keep]).astype(np.float64)
    qf = G.bf16_to_f32(q).astype(np.float64)
    for h in range(hq):
        w = np.exp((kd @ qf[0, h]) * scale - ((kd @ qf[0, h]) * scale).max())
        np.testing.assert_allclose(out[0, h], (w @ vd) / w.sum(), rtol=1e-12)
    holed[0, :] = -1
    assert not G.decode_attention(q, c, holed, mb, np.array([64]), -1, hq, hkv, scale).any()
    assert not G.rows_attention(q, np.array([63]), np.array([0]), c, holed, mb, 1, -1, hq, hkv, scale).any()
