"""numpy restatement of the fp8-KV decode path (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Every function states the rule it fixes and the reference file:line it follows. The reference caches K/V in bf16
(model/kernels/decode.cu:4-7); the fp8 scheme (per-token, per-kv-head absmax scale, OCP e4m3fn) is defined by the
benchmark configuration, not by the reference, and is restated here as the build's spec.

Layout spec shared with the HIP kernels (nanochat_amd/csrc/layout.h): one byte pool [num_blocks][Hkv][4224]; the
(block, kv head) tile holds, in four 1 KiB parts of 64 16-byte fragments (fragment f at part*1024 + 16 f),
  [0, 2048)     K codes: key t, dim d at ((d/16)%2)*1024 + (t + 16 (d/32))*16 + d%16
  [2048, 4096)  V codes, quad-transposed: key t, dim d at 2048 + ((d/4)%2)*1024 + (d/8 + 16 (t/4))*16 + (d%4)*4 + t%4
  [4096, 4160)  K scales fp32 [16], one per (token, kv head)
  [4160, 4224)  V scales fp32 [16]
  block table int32 [B][max_blocks]; None means contiguous: sequence b's page i is block b*max_blocks + i.
"""

from __future__ import annotations

import numpy as np

HEAD_DIM = 128
HALF = HEAD_DIM // 2
PAGE = 16
FP8_MAX = np.float32(448.0)
# model/ops/linear.py:20 EPS = torch.finfo(torch.float32).eps, the RMS norms' epsilon (also qk_row.cuh:30)
EPS = np.float32(np.finfo(np.float32).eps)


# ---------------------------------------------------------------------------------------------------------------
# rounding primitives
# ---------------------------------------------------------------------------------------------------------------

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits (uint16), round to nearest even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bits (uint16) -> fp32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> OCP float8 e4m3fn code (uint8), round to nearest even, no saturation: |x| > 464 (and inf, NaN) give
    the NaN code 0x7F | sign, exactly as torch's float32 -> float8_e4m3fn cast (tests pin it against torch).
    Normal results (|x| >= 2^-6): re-bias the fp32 exponent by 127 - 7 and round the 23-bit mantissa to 3 bits;
    subnormal results: rint(|x| * 2^9), the count of 2^-9 steps (8 of them is the smallest normal, code 0x08)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.int64)
    a = (u & 0x7FFFFFFF).astype(np.int64)
    v = a - (120 << 23)
    normal = (v + 0x7FFFF + ((v >> 20) & 1)) >> 20
    small = np.minimum(np.abs(np.nan_to_num(x)), np.float32(1.0))  # the subnormal branch only reads |x| < 2^-6
    sub = np.rint(small * np.float32(512.0)).astype(np.int64)
    code = np.where(a >= 0x3C800000, normal, sub)
    code = np.where((code > 0x7E) | (a >= 0x7F800000), 0x7F, code)
    return (code | sign).astype(np.uint8)


def e4m3_decode(c: np.ndarray) -> np.ndarray:
    """OCP float8 e4m3fn code -> fp32 (exact): e = 0 subnormal m 2^-9, else (1 + m/8) 2^(e-7); 0x7F/0xFF NaN."""
    c = np.asarray(c, dtype=np.uint8).astype(np.int64)
    e, m = (c >> 3) & 0xF, c & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(c & 0x80, -mag, mag).astype(np.float32)


E4M3_TABLE = e4m3_decode(np.arange(256, dtype=np.uint8))


# ---------------------------------------------------------------------------------------------------------------
# rotary tables and the q/k row math
# ---------------------------------------------------------------------------------------------------------------

def rotary_tables(n: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """cos, sin fp32 [n][64] of t theta^(-2i/128), computed in fp64 and rounded once (model/modeling.py:169-176,
    inference/modeling_nanochat.py:29-34)."""
    exponent = np.arange(0, HEAD_DIM, 2, dtype=np.float64) / HEAD_DIM
    freqs = np.outer(np.arange(n, dtype=np.float64), float(theta) ** -exponent)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


def sum_squares(x: np.ndarray) -> np.ndarray:
    """Σ x_i² over the last axis (128) in the build's fixed fp32 tree, every product and add rounded, no FMA:
    pairs (i, i+64) first; the 64 sums as 8 groups of 8 consecutive (i = 8g + e) halved in place (e, e+4), (e, e+2),
    (e, e+1); then the 8 group sums halved (g, g+4), (g, g+2), (g, g+1). A group is one lane of an 8-lane row in
    the HIP kernels (qk_row.h), so the last three levels are xor-4/2/1 lane exchanges."""
    sq = x * x
    s = sq[..., :HALF] + sq[..., HALF:]
    a = s.reshape(*s.shape[:-1], 8, 8)
    a = a[..., :4] + a[..., 4:]
    a = a[..., :2] + a[..., 2:]
    a = a[..., 0] + a[..., 1]
    a = a[..., :4] + a[..., 4:]
    a = a[..., :2] + a[..., 2:]
    return a[..., 0] + a[..., 1]


def qk_norm_rope(x_bits: np.ndarray, gain: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """bf16 rows [..., 128] -> bf16 bits: n = x r g with r = 1 / sqrt(Σx²/128 + FLT_EPSILON) (correctly rounded sqrt
    and division, the tree of sum_squares), then the rotation by -θ of pairs (i, i+64): y1 = n1 c + n2 s,
    y2 = n2 c - n1 s, every operation one fp32 rounding, no FMA; one bf16 rounding at the end.
    Follows model/kernels/qk_row.cuh:25-41 (norm -> gain -> rotate) and inference/modeling_nanochat.py:37-45;
    cos, sin broadcast against x's leading axes ([..., 64])."""
    x = bf16_to_f32(x_bits)
    r = np.float32(1.0) / np.sqrt(sum_squares(x) / np.float32(HEAD_DIM) + EPS)
    n = (x * r[..., None]) * np.asarray(gain, dtype=np.float32)
    n1, n2 = n[..., :HALF], n[..., HALF:]
    y = np.concatenate([n1 * cos + n2 * sin, n2 * cos - n1 * sin], axis=-1)
    return bf16_bits(y)


def quantize_rows(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """bf16 rows [..., 128] -> (e4m3fn codes uint8 [..., 128], fp32 scale [...]): a = max |x| (exact),
    scale = a / 448 (fp32 division), code = e4m3(x / scale); an all-zero row stores scale 0 and codes 0."""
    x = bf16_to_f32(x_bits)
    a = np.abs(x).max(axis=-1)
    scale = (a / FP8_MAX).astype(np.float32)
    safe = np.where(scale == 0, np.float32(1.0), scale)
    codes = e4m3_encode(x / safe[..., None])
    codes = np.where((scale == 0)[..., None], np.uint8(0), codes)
    return codes, scale


def dequantize(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """fp32(code) * scale, one fp32 rounding."""
    return E4M3_TABLE[codes] * np.asarray(scale, dtype=np.float32)[..., None]


# ---------------------------------------------------------------------------------------------------------------
# the paged cache
# ---------------------------------------------------------------------------------------------------------------

TILE_BYTES = 4224


def k_byte(t, d):
    """Byte of key t, dim d in a tile (module docstring)."""
    return ((d // 16) % 2) * 1024 + (t + 16 * (d // 32)) * 16 + d % 16


def v_byte(t, d):
    """Byte of key t, dim d in a tile (module docstring)."""
    return 2048 + ((d // 4) % 2) * 1024 + (d // 8 + 16 * (t // 4)) * 16 + (d % 4) * 4 + t % 4


_T, _D = np.meshgrid(np.arange(PAGE), np.arange(HEAD_DIM), indexing="ij")
K_BYTES = k_byte(_T, _D)  # [16][128]
V_BYTES = v_byte(_T, _D)


class PagedCache:
    """The HIP kernels' cache layout (module docstring): the byte pool `pages`, its codes at K_BYTES / V_BYTES
    [t][d] of a tile, and views of the scales (k_scale / v_scale fp32 [nb][Hkv][16]); writes land in the pool."""

    def __init__(self, num_blocks: int, hkv: int):
        self.num_blocks, self.hkv = num_blocks, hkv
        self.pages = np.zeros((num_blocks, hkv, TILE_BYTES), np.uint8)
        self.k_scale = self.pages[..., 4096:4160].view(np.float32)
        self.v_scale = self.pages[..., 4160:4224].view(np.float32)
        assert all(np.shares_memory(x, self.pages) for x in (self.k_scale, self.v_scale))

    @staticmethod
    def block_of(seq: np.ndarray, pos: np.ndarray, block_table: np.ndarray | None, max_blocks: int) -> np.ndarray:
        seq, pos = np.asarray(seq, np.int64), np.asarray(pos, np.int64)
        if block_table is None:
            return seq * max_blocks + pos // PAGE
        return np.asarray(block_table, np.int64)[seq, pos // PAGE]

    def write(self, blk, head, t, k_codes, k_scale, v_codes, v_scale) -> None:
        """Rows (codes [..][128] in dim order) for (block, kv head, token-in-page) index arrays (broadcast)."""
        blk, head, t = np.broadcast_arrays(np.asarray(blk), np.asarray(head), np.asarray(t))
        self.pages[blk[..., None], head[..., None], K_BYTES[t]] = k_codes
        self.pages[blk[..., None], head[..., None], V_BYTES[t]] = v_codes
        self.k_scale[blk, head, t] = k_scale
        self.v_scale[blk, head, t] = v_scale

    def read(self, blk, head, t) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
        """(K codes, V codes in dim order, K scale, V scale) at index arrays blk, head, t (broadcast)."""
        blk, head, t = np.broadcast_arrays(np.asarray(blk), np.asarray(head), np.asarray(t))
        return (self.pages[blk[..., None], head[..., None], K_BYTES[t]],
                self.pages[blk[..., None], head[..., None], V_BYTES[t]], self.k_scale[blk, head, t],
                self.v_scale[blk, head, t])


def append(cache: PagedCache, qkv_bits: np.ndarray, pos: np.ndarray, seq: np.ndarray, q_gain: np.ndarray,
           k_gain: np.ndarray, cos: np.ndarray, sin: np.ndarray, hq: int, hkv: int,
           block_table: np.ndarray | None, max_blocks: int) -> np.ndarray:
    """Append n rows of the fused projection (bf16 [n][(hq + 2 hkv) 128]: q heads, k heads, v heads) at positions
    pos[n] of sequences seq[n]: q and k through qk_norm_rope at their position (decode.cu:495-505), v as is
    (decode.cu:494); k and v quantised per (token, kv head) and written to the cache (decode.cu:562-564 writes bf16;
    here fp8 + scale). Returns q_out bf16 bits [n][hq][128]."""
    n = qkv_bits.shape[0]
    D = HEAD_DIM
    heads = qkv_bits[:, :(hq + 2 * hkv) * D].reshape(n, hq + 2 * hkv, D)
    c, s = cos[pos][:, None, :], sin[pos][:, None, :]
    q_out = qk_norm_rope(heads[:, :hq], q_gain, c, s)
    k_bits = qk_norm_rope(heads[:, hq:hq + hkv], k_gain, c, s)
    v_bits = heads[:, hq + hkv:]
    kc, ks = quantize_rows(k_bits)
    vc, vs = quantize_rows(v_bits)
    blk = PagedCache.block_of(seq, pos, block_table, max_blocks)
    t = np.asarray(pos, np.int64) % PAGE
    for h in range(hkv):
        cache.write(blk, h, t, kc[:, h], ks[:, h], vc[:, h], vs[:, h])
    return q_out


def gather(cache: PagedCache, block_table: np.ndarray | None, max_blocks: int, ctx_len: np.ndarray,
           max_ctx: int) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """Each sequence's first ctx_len[b] positions in the canonical row-major layout: K, V codes uint8
    [B][Hkv][max_ctx][128], scales fp32 [B][Hkv][max_ctx]; positions past ctx_len are zero."""
    B, H = len(ctx_len), cache.hkv
    k = np.zeros((B, H, max_ctx, HEAD_DIM), np.uint8)
    v = np.zeros_like(k)
    ks = np.zeros((B, H, max_ctx), np.float32)
    vs = np.zeros_like(ks)
    for b in range(B):
        t = np.arange(int(ctx_len[b]))
        blk = PagedCache.block_of(np.full_like(t, b), t, block_table, max_blocks)
        for h in range(H):
            k[b, h, :len(t)], v[b, h, :len(t)], ks[b, h, :len(t)], vs[b, h, :len(t)] = cache.read(blk, h, t % PAGE)
    return k, v, ks, vs


ROW_BYTES = 2 * HEAD_DIM + 8  # a position of a kv head as a row: K codes, V codes, K scale, V scale


def export_rows(cache: PagedCache, block_table: np.ndarray | None, max_blocks: int, seq: int, at: int,
                n: int) -> np.ndarray:
    """Positions [at, at + n) of sequence seq as rows uint8 [n][Hkv][264]: K codes, V codes in dim order, then the K
    and V scales' fp32 bytes; a position whose block is missing (< 0 or past the pool) gives a zero row. The prompt
    store's unit: the reference copies a slot's positions [at, at + n) to the store position by position
    (model/kernels/decode.cu:1053-1075, bf16 K and V rows there)."""
    rows = np.zeros((n, cache.hkv, ROW_BYTES), np.uint8)
    for i in range(n):
        blk = _block_or_missing(cache, block_table, max_blocks, seq, at + i)
        if blk < 0:
            continue
        for h in range(cache.hkv):
            kc, vc, ks, vs = cache.read(blk, h, (at + i) % PAGE)
            rows[i, h] = np.concatenate([kc, vc, np.array([ks, vs], np.float32).view(np.uint8)])
    return rows


def import_rows(cache: PagedCache, rows: np.ndarray, block_table: np.ndarray | None, max_blocks: int, seq: int,
                at: int) -> None:
    """export_rows' inverse (the store-to-slot direction of decode.cu:1053-1075): rows [n][Hkv][264] into positions
    [at, at + n) of sequence seq; a position whose block is missing is not written."""
    for i in range(rows.shape[0]):
        blk = _block_or_missing(cache, block_table, max_blocks, seq, at + i)
        if blk < 0:
            continue
        for h in range(cache.hkv):
            r = rows[i, h]
            sc = r[2 * HEAD_DIM:].view(np.float32)
            cache.write(blk, h, (at + i) % PAGE, r[:HEAD_DIM], sc[0], r[HEAD_DIM:2 * HEAD_DIM], sc[1])


def _block_or_missing(cache: PagedCache, block_table, max_blocks: int, seq: int, pos: int) -> int:
    page = pos // PAGE
    if page >= max_blocks:
        return -1
    blk = int(PagedCache.block_of(seq, pos, block_table, max_blocks))
    return blk if 0 <= blk < cache.num_blocks else -1


# ---------------------------------------------------------------------------------------------------------------
# attention (fp64 over the dequantised cache)
# ---------------------------------------------------------------------------------------------------------------

def key_range(p: int, window: int) -> tuple[int, int]:
    """Keys [begin, p] of the query at position p: `window` keys before it at most (decode.cu:575), all if window < 0
    (a full layer's window is the context, model/modeling.py:40-44)."""
    begin = 0 if window < 0 or p <= window else p - window
    return begin, p + 1


def _kv_dequantized(cache: PagedCache, b: int, h: int, lo: int, hi: int, block_table, max_blocks):
    """Dequantised K, V of keys [lo, hi) of sequence b, kv head h, and which keys have a block (a page past
    max_blocks, or a table entry outside [0, num_blocks), has none: its keys are skipped, as by the kernels'
    lookup_block)."""
    t = np.arange(lo, hi)
    page = t // PAGE
    present = page < max_blocks
    if block_table is None:
        blk = b * max_blocks + page
    else:
        blk = np.asarray(block_table, np.int64)[b, np.minimum(page, max_blocks - 1)]
    present &= (blk >= 0) & (blk < cache.num_blocks)
    blk = np.where(present, blk, 0)
    kc, vc, ks, vs = cache.read(blk, h, t % PAGE)
    return dequantize(kc, ks).astype(np.float64), dequantize(vc, vs).astype(np.float64), present


def softmax_attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, mask: np.ndarray | None = None):
    """softmax(q kᵀ scale [+ mask]) v in fp64; q [m][128], k, v [n][128]; mask True = excluded. A row with every
    key excluded is zero."""
    s = (q @ k.T) * scale
    if mask is not None:
        s = np.where(mask, -np.inf, s)
    top = s.max(axis=-1, keepdims=True)
    empty = ~np.isfinite(top)
    p = np.exp(s - np.where(empty, 0.0, top))
    den = p.sum(axis=-1, keepdims=True)
    return np.where(empty, 0.0, (p @ v) / np.where(empty, 1.0, den))


def decode_attention(q_bits: np.ndarray, cache: PagedCache, block_table: np.ndarray | None, max_blocks: int,
                     ctx_len: np.ndarray, window: int, hq: int, hkv: int, sm_scale: float) -> np.ndarray:
    """Single-query attention (decode.cu:567-675; Appendix rule: keys [max(p - window, 0), p] from the cache, the
    query's own key included, p = ctx_len - 1), query head h reading kv head h / (hq / hkv); fp64 [B][hq][128]."""
    B = q_bits.shape[0]
    G = hq // hkv
    q = bf16_to_f32(q_bits).astype(np.float64)
    out = np.zeros((B, hq, HEAD_DIM), np.float64)
    for b in range(B):
        lo, hi = key_range(int(ctx_len[b]) - 1, window)
        for h in range(hkv):
            k, v, present = _kv_dequantized(cache, b, h, lo, hi, block_table, max_blocks)
            out[b, h * G:(h + 1) * G] = softmax_attend(q[b, h * G:(h + 1) * G], k, v, sm_scale, ~present[None, :])
    return out


def prefill_attention(q_bits: np.ndarray, cu_q: np.ndarray, q_start: np.ndarray, cache: PagedCache,
                      block_table: np.ndarray | None, max_blocks: int, window: int, hq: int, hkv: int,
                      sm_scale: float) -> np.ndarray:
    """Chunked prefill (decode.cu:859-861 ordering; Appendix rule 5): rows cu_q[b]..cu_q[b+1] of sequence b sit at
    positions q_start[b] + i and, after the whole chunk is appended, attend keys [max(p - window, 0), p] of the fp8
    cache; fp64 [n][hq][128]."""
    G = hq // hkv
    q = bf16_to_f32(q_bits).astype(np.float64)
    out = np.zeros(q.shape, np.float64)
    for b in range(len(q_start)):
        r0, r1 = int(cu_q[b]), int(cu_q[b + 1])
        if r1 == r0:
            continue
        p = int(q_start[b]) + np.arange(r1 - r0)
        lo = min(key_range(int(x), window)[0] for x in p)
        hi = int(p[-1]) + 1
        keys = np.arange(lo, hi)
        begin = np.array([key_range(int(x), window)[0] for x in p])
        mask = (keys[None, :] > p[:, None]) | (keys[None, :] < begin[:, None])
        for h in range(hkv):
            k, v, present = _kv_dequantized(cache, b, h, lo, hi, block_table, max_blocks)
            for g in range(G):
                out[r0:r1, h * G + g] = softmax_attend(q[r0:r1, h * G + g], k, v, sm_scale, mask | ~present)
    return out


def rows_attention(q_bits: np.ndarray, pos: np.ndarray, seq: np.ndarray, cache: PagedCache,
                   block_table: np.ndarray | None, max_blocks: int, num_seqs: int, window: int, hq: int, hkv: int,
                   sm_scale: float) -> np.ndarray:
    """Prefill attention over arbitrary rows (dec_prefill's rows, decode.cu:1039-1051, each a k_attn query): row r
    at position pos[r] of sequence seq[r] attends keys [max(p - window, 0), p] of the fp8 cache; rows with
    pos < 0 or seq outside [0, num_seqs) are zero; fp64 [n][hq][128]."""
    G = hq // hkv
    q = bf16_to_f32(q_bits).astype(np.float64)
    out = np.zeros(q.shape, np.float64)
    valid = (pos >= 0) & (seq >= 0) & (seq < num_seqs)
    for s in np.unique(seq[valid]):
        rows = np.nonzero(valid & (seq == s))[0]
        p = pos[rows].astype(np.int64)
        begin = np.array([key_range(int(x), window)[0] for x in p])
        lo, hi = int(begin.min()), int(p.max()) + 1
        keys = np.arange(lo, hi)
        mask = (keys[None, :] > p[:, None]) | (keys[None, :] < begin[:, None])
        for h in range(hkv):
            k, v, present = _kv_dequantized(cache, int(s), h, lo, hi, block_table, max_blocks)
            for g in range(G):
                out[rows, h * G + g] = softmax_attend(q[rows, h * G + g], k, v, sm_scale, mask | ~present)
    return out
