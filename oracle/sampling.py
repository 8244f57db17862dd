"""numpy restatement of the decode step's token choice (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

The reference chooses each slot's next token in the lm_head GEMM's ARGMAX epilogue and k_nucleus, then commits it
in k_commit (model/kernels/decode.cu:90-105,170-209,360-404,676-689); the host side is inference/decoder.py:28-40
(temperature 0: argmax, ties to the lowest id; > 0: a softmax(logits / temperature) sample drawn from (seed,
generated position) alone; top_p < 1: nucleus sampling). Per active slot b:

  allowed(r)  every row, or for a masked slot the rows whose bit r % 32 of word r // 32 of its allow row is set
  T == 0      score = s (the raw fp32 logit), the choice = the largest score over allowed rows, lowest row on ties
  T > 0       z = c tanh(s / c) (the logit cap c; none for c <= 0), score = z / T + gumbel(seed, i, r),
              i = pos - first (the generated token's index): the Gumbel-max sample of softmax(z / T)
              (arXiv 1411.0030 §2)
  top_p < 1   (T > 0) nucleus (arXiv 1904.09751 §3.1; transformers' TopPLogitsWarper): e = exp(z / T - max),
              keep e >= e*, e* the least e with sum(e' <= e*) > (1 - top_p) sum(e) (ties kept or dropped together),
              then the Gumbel-max choice over the kept rows
  alt         the best allowed row but `lazy` (the row the host may reject), none for a nucleus slot
  commit      token = the choice's row (-1 if no row was allowed), alt token likewise, pos += 1

The packed key (decode.cu:90-96): the score's IEEE bits mapped to an unsigned order, then ~row; the largest key holds
the largest score and the lowest row among exact ties. Philox4x32-10 is restated from its published definition
(Salmon et al., "Parallel random numbers: as easy as 1, 2, 3", SC '11) and pinned by that paper's known-answer
vectors (tests/test_oracle_sampling.py); the Gumbel transform follows decode.cu:98-105: the top 52 bits r of the
first two output words, u = (2r + 1) 2^-53 in (0, 1), g = float(-log(-log(u))) in float64.
"""

from __future__ import annotations

import numpy as np

PHILOX_M = (0xD2511F53, 0xCD9E8D57)      # round multipliers (SC '11, Philox4x32)
PHILOX_W = (0x9E3779B9, 0xBB67AE85)      # key schedule increments (golden ratio, sqrt(3) - 1)


def philox4x32_10(ctr, key) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """Philox4x32 with 10 rounds, vectorised: ctr 4 uint32 arrays (or ints), key 2. Each round: (hi0, lo0) = M0 c0,
    (hi1, lo1) = M1 c2 (32x32 -> 64-bit products), c = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0); the key advances by
    the increments between rounds."""
    c = [np.asarray(x, dtype=np.uint32) for x in ctr]
    k0, k1 = (np.asarray(x, dtype=np.uint32) for x in key)
    m0, m1 = np.uint64(PHILOX_M[0]), np.uint64(PHILOX_M[1])
    with np.errstate(over="ignore"):
        for r in range(10):
            p0 = m0 * c[0].astype(np.uint64)
            p1 = m1 * c[2].astype(np.uint64)
            hi0, lo0 = (p0 >> np.uint64(32)).astype(np.uint32), p0.astype(np.uint32)
            hi1, lo1 = (p1 >> np.uint64(32)).astype(np.uint32), p1.astype(np.uint32)
            c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
            if r < 9:
                k0 = (k0 + np.uint32(PHILOX_W[0])).astype(np.uint32)
                k1 = (k1 + np.uint32(PHILOX_W[1])).astype(np.uint32)
    return c[0], c[1], c[2], c[3]


def gumbel(seed: int, i: int, rows: np.ndarray) -> np.ndarray:
    """Gumbel noise of rows at sample index i (decode.cu:98-105): counter (row, i, 0, 0), key (seed low, seed high)."""
    rows = np.asarray(rows, dtype=np.uint32)
    z = np.zeros_like(rows)
    x0, x1, _, _ = philox4x32_10((rows, np.full_like(rows, np.uint32(i & 0xFFFFFFFF)), z, z),
                                 (np.uint32(seed & 0xFFFFFFFF), np.uint32((seed >> 32) & 0xFFFFFFFF)))
    r = ((x0.astype(np.uint64) << np.uint64(32)) | x1.astype(np.uint64)) >> np.uint64(12)
    u = (2.0 * r.astype(np.float64) + 1.0) * 2.0 ** -53
    return (-np.log(-np.log(u))).astype(np.float32)


def choice_key(score: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """(ordered score bits) << 32 | ~row, uint64 (decode.cu:90-96)."""
    bits = np.ascontiguousarray(score, dtype=np.float32).view(np.uint32).astype(np.uint64)
    ordered = np.where(bits & 0x80000000, ~bits & 0xFFFFFFFF, bits | 0x80000000)
    return (ordered << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - np.asarray(rows, dtype=np.uint64))


def key_row(key: int) -> int:
    """The row of a packed key, -1 for the empty key 0 (k_commit, decode.cu:683-684)."""
    return int(np.int32(np.uint32(0xFFFFFFFF - (int(key) & 0xFFFFFFFF))))


def capped(s: np.ndarray, softcap: float) -> np.ndarray:
    """c tanh(s / c) in fp32 (decode.cu:195), or s for c <= 0."""
    s = np.asarray(s, dtype=np.float32)
    if softcap <= 0:
        return s
    c = np.float32(softcap)
    return (c * np.tanh(s / c)).astype(np.float32)


def nucleus_keep(e: np.ndarray, top_p: float) -> np.ndarray:
    """Rows kept by nucleus sampling: e >= e*, e* the least value with sum(e' <= e*) > (1 - top_p) sum(e), sums in
    float64 (k_nucleus's bisection over the IEEE bits of e*, decode.cu:380-392). top_p <= 0 keeps the largest."""
    e = np.asarray(e, dtype=np.float32)
    total = float(np.sum(e, dtype=np.float64))
    drop = float(np.float32(np.float32(1.0) - np.float32(top_p)) * np.float32(total))
    vals, inv = np.unique(e, return_inverse=True)
    mass = np.bincount(inv, weights=e.astype(np.float64), minlength=len(vals))
    cum = np.cumsum(mass)
    over = np.nonzero(cum > drop)[0]
    least = vals[over[0]] if len(over) else np.float32(1.0)
    return e >= least


def choose(logits: np.ndarray, *, temperature: np.ndarray, top_p: np.ndarray, seed: np.ndarray, pos: np.ndarray,
           first: np.ndarray, active: np.ndarray | None = None, masked: np.ndarray | None = None,
           allow: np.ndarray | None = None, softcap: float = 15.0, lazy: int = -1
           ) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Every active slot's choice and alternative, and the committed positions. logits fp32 [B][vocab]; per slot
    temperature, top_p (fp32), seed (uint64), pos, first (int32); active / masked bool [B] (None: all active, none
    masked); allow uint32 [B][ceil(vocab / 32)]. Returns (tokens, alt_tokens, pos) with inactive slots' entries -2
    (unwritten) and their positions unchanged."""
    logits = np.asarray(logits, dtype=np.float32)
    B, V = logits.shape
    active = np.ones(B, bool) if active is None else np.asarray(active, bool)
    masked = np.zeros(B, bool) if masked is None else np.asarray(masked, bool)
    tokens = np.full(B, -2, np.int32)
    alts = np.full(B, -2, np.int32)
    pos_out = np.asarray(pos, dtype=np.int32).copy()
    rows = np.arange(V)
    for b in range(B):
        if not active[b]:
            continue
        ok = np.ones(V, bool)
        if masked[b]:
            words = np.asarray(allow[b], dtype=np.uint32)
            ok = ((words[rows // 32] >> (rows % 32).astype(np.uint32)) & 1).astype(bool)
        s = logits[b]
        T = np.float32(temperature[b])
        i = int(pos[b]) - int(first[b])
        best = alt = 0
        if T > 0 and np.float32(top_p[b]) < 1:
            z = np.where(ok, capped(s, softcap), np.float32(-np.inf)).astype(np.float32)
            zt = (z / T).astype(np.float32)
            m = np.max(zt)
            with np.errstate(invalid="ignore"):  # no allowed row: m = -inf, nothing kept below
                e = np.where(ok, np.exp((zt - m).astype(np.float32)), np.float32(0)).astype(np.float32)
            keep = nucleus_keep(e, float(top_p[b])) & ok
            if keep.any():
                kr = rows[keep]
                score = (zt[keep] + gumbel(int(seed[b]), i, kr)).astype(np.float32)
                best = int(choice_key(score, kr).max())
        elif ok.any():
            kr = rows[ok]
            if T > 0:
                score = ((capped(s[ok], softcap) / T).astype(np.float32) + gumbel(int(seed[b]), i, kr))
            else:
                score = s[ok]
            keys = choice_key(np.asarray(score, np.float32), kr)
            best = int(keys.max())
            not_lazy = kr != lazy
            alt = int(keys[not_lazy].max()) if not_lazy.any() else 0
        tokens[b] = key_row(best)
        alts[b] = key_row(alt)
        pos_out[b] += 1
    return tokens, alts, pos_out
