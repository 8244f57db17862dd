/*
 * nanochat_amd: the C ABI of the MI355X (gfx950) fp8-KV decode path, libnanochat_amd.so.
 *
 * Conventions (the reference's, model/kernels/*.cu with native.py:43-65): every tensor is a raw device pointer,
 * counts are C ints, the HIP stream is the last argument, and every launch is stream-ordered and asynchronous.
 * Two error classes:
 *   - argument errors are checked on the host before any launch: the call returns a negative status and
 *     nc_last_error() names the problem (the reference validates in Python, inference/decoder.py:197-201);
 *   - a failed HIP runtime call or launch aborts the process with file:line (model/kernels/decode.cu:47-53).
 * Device-side, rows or keys whose position, sequence or block is out of range are skipped, never written or read
 * out of bounds.
 *
 * Cache layout (per layer), PAGE = 16 positions per block, D = 128: one pool, uint8 [num_blocks][Hkv][4224]; the
 * (block, kv head) tile is
 *   [0, 2048)     K codes [16][128], row-major
 *   [2048, 4096)  V codes, quad-transposed: key t, dim d at 2048 + (t/4)*512 + d*4 + t%4
 *   [4096, 4160)  K scales fp32 [16], one absmax/448 scale per (token, kv head)
 *   [4160, 4224)  V scales fp32 [16]
 *   block_table int32 [num_seqs][max_blocks], or NULL: contiguous, sequence s's page i is block s*max_blocks + i
 * Codes are OCP float8 e4m3fn, rounded to nearest even from x / scale; the reference caches bf16 instead
 * (model/kernels/decode.cu:4-7, 726).
 */
#ifndef NANOCHAT_AMD_H
#define NANOCHAT_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of this header (1). */
int nc_abi_version(void);

/* Message of the last failed call on this thread. */
const char *nc_last_error(void);

/* Training-layout q/k prologue: RMS norm with fp32 gains gq, gk (128), then RoPE by cos/sin fp32 [T][64] at
 * position t % T. q, k: bf16 (B, T, H, 128) column blocks of a (B, T, 3 H 128) projection; qo, ko: contiguous
 * bf16 (B, T, H, 128); rows = B T H.
 * Replaces: qkp_forward, model/kernels/qk_prologue.cu:111-118 (same signature); called by qk_forward,
 * model/ops/qk_prologue.py:13-21. */
void qkp_forward(const void *q, const void *k, const void *gq, const void *gk, void *qo, void *ko, const void *cos,
                 const void *sin, long long rows, int H, int T, void *stream);

/* Fused append of n rows of the fused projection qkv (bf16 [n][row_stride]: Hq q heads, Hkv k heads, Hkv v heads
 * of 128): q and k RMS-normed with gains q_gain, k_gain, rotated by cos/sin fp32 [rope_len][64] at pos[n]; q to
 * q_out (bf16 [n][Hq][128]); k and v quantised per (token, kv head) into sequence seq[n]'s page. A row out of range
 * (pos < 0 or >= rope_len or past max_blocks pages, seq outside [0, num_seqs), block outside [0, num_blocks))
 * writes no cache byte and gets a NaN q_out row. ctx_out (optional, int32 [n], must not overlap pos) receives
 * pos + 1 for every row: the context lengths the following decode attends with, and the next step's positions
 * (the position advance the reference's k_commit makes, decode.cu:1107-1124, without a kernel of its own).
 * Replaces: k_prologue + attn_prologue, model/kernels/decode.cu:476-507,550-565 (which cache bf16). */
int nc_kv_append_fp8(const void *qkv, long long row_stride, int n, const int32_t *pos, const int32_t *seq,
                     const float *q_gain, const float *k_gain, const float *cos, const float *sin, int rope_len,
                     int hq, int hkv, void *q_out, uint8_t *cache, const int32_t *block_table, int max_blocks,
                     int num_blocks, int num_seqs, int32_t *ctx_out, void *stream);

/* Quantise-and-store of final K and V rows (bf16 [n][row_stride], Hkv heads of 128, no norm or rotation) at
 * (seq[n], pos[n]).
 * Replaces: the cache write of DynamicCache.update, inference/modeling_nanochat.py:95-96 (bf16 there). */
int nc_kv_store_fp8(const void *k, const void *v, long long row_stride, int n, const int32_t *pos,
                    const int32_t *seq, int hkv, uint8_t *cache, const int32_t *block_table, int max_blocks,
                    int num_blocks, int num_seqs, void *stream);

/* Gather of sequences 0..B-1: codes of the first ctx_len[b] positions to k_out, v_out (uint8
 * [B][Hkv][max_ctx][128], both row-major) and scales to ks_out, vs_out (fp32 [B][Hkv][max_ctx]); later
 * positions are zero.
 * Replaces: the contiguous per-slot cache read of k_attn's load_run, model/kernels/decode.cu:581-591, and the
 * prompt copies of prompt_copy, decode.cu:1053-1067. */
int nc_kv_gather_fp8(const uint8_t *cache, const int32_t *block_table, int max_blocks, int num_blocks,
                     const int32_t *ctx_len, int B, int hkv, int max_ctx, uint8_t *k_out, uint8_t *v_out,
                     float *ks_out, float *vs_out, void *stream);

/* Workspace bytes nc_decode_attn_fp8 needs for B sequences of hq / hkv heads (independent of max_ctx and of the
 * device): a partial-result slot (Σ p v, max, sum) per wave and per (sequence, kv head). */
long long nc_decode_workspace_bytes(int B, int hq, int hkv, int max_ctx);

/* Single-token decode attention: query b (bf16 q [B][Hq][128]) at position p = ctx_len[b] - 1 attends keys
 * [max(p - window, 0), p] of sequence b (window < 0: all), query head h reading kv head h / (Hq / Hkv), scores
 * times sm_scale, fp32 softmax, bf16 out [B][Hq][128]. ctx_len values above max_ctx are clamped to it; a
 * sequence with ctx_len <= 0 gets a zero row. Hq / Hkv <= 16. The workspace (nc_decode_workspace_bytes) holds
 * partial results between the call's two kernels: calls in one stream may share it, calls that may overlap (two
 * streams) need one each. The pool's code bytes must be valid e4m3fn codes (a zero-initialised pool written only
 * by nc_kv_append_fp8 / nc_kv_store_fp8 is).
 * Replaces: k_attn, model/kernels/decode.cu:567-675 (bf16 MHA, one block per (head, slot)). */
int nc_decode_attn_fp8(const void *q, const uint8_t *cache, const int32_t *block_table, int max_blocks,
                       int num_blocks, const int32_t *ctx_len, int window, int B, int hq, int hkv, int max_ctx,
                       float sm_scale, void *out, void *workspace, long long workspace_bytes, void *stream);

/* A whole decode step's attention in two launches: the append of nc_kv_append_fp8 fused into
 * nc_decode_attn_fp8. Row b of the projection qkv (bf16 [B][row_stride]: Hq q heads, Hkv k heads, Hkv v heads)
 * is token pos[b] of sequence b: its q heads are QK-normed, gained (q_gain [128]) and rotated (cos / sin
 * [rope_len][64]) as nc_kv_append_fp8 does, its key (k_gain) and value are quantised into sequence b's page, and
 * q attends keys [max(pos - window, 0), pos], the new key included. Cache bytes, scales and out are bit-identical
 * to nc_kv_append_fp8 (seq[b] = b) followed by nc_decode_attn_fp8 with ctx_len = pos + 1, for every row with
 * 0 <= pos < min(max_ctx, rope_len). A row with pos < 0 writes nothing and gets a zero row; a row with pos at or
 * past max_ctx or rope_len writes nothing and gets a NaN row. pos_out (optional, int32 [B], not overlapping pos)
 * receives pos + 1, the next step's positions. out must not overlap qkv. Workspace and other arguments as
 * nc_decode_attn_fp8.
 * Replaces: the decode body's k_prologue append (model/kernels/decode.cu:550-565) and k_attn (decode.cu:567-675),
 * launched back to back by the reference. */
int nc_decode_step_fp8(const void *qkv, long long row_stride, const int32_t *pos, int32_t *pos_out,
                       const float *q_gain, const float *k_gain, const float *cos, const float *sin, int rope_len,
                       uint8_t *cache, const int32_t *block_table, int max_blocks, int num_blocks, int window, int B,
                       int hq, int hkv, int max_ctx, float sm_scale, void *out, void *workspace,
                       long long workspace_bytes, void *stream);

/* Chunked-prefill attention: row r (bf16 q [n][Hq][128], normed and rotated, e.g. nc_kv_append_fp8's q_out) at
 * position pos[r] of sequence seq[r] attends keys [max(pos - window, 0), pos] of that sequence in the cache
 * (window < 0: all), query head h reading kv head h / (Hq / Hkv), scores times sm_scale, fp32 softmax, bf16 out
 * [n][Hq][128]. The rows' own keys must be in the cache already (append the whole chunk first), so each row sees
 * the chunk's earlier rows causally. Rows with pos < 0 or seq outside [0, num_seqs) get zero rows; keys of a
 * missing block are skipped. Rows may come in any order; a sequence's rows being consecutive is fastest.
 * Hq / Hkv <= 16.
 * Replaces: dec_prefill, model/kernels/decode.cu:1039-1051, whose rows each run k_attn (decode.cu:567-675). */
int nc_prefill_attn_fp8(const void *q, const int32_t *pos, const int32_t *seq, int n, const uint8_t *cache,
                        const int32_t *block_table, int max_blocks, int num_blocks, int num_seqs, int window, int hq,
                        int hkv, float sm_scale, void *out, void *stream);

/* Greedy token choice: out[r] = the column of the largest fp32 logit of row r (logits [rows][ld], cols used), the
 * lowest column among exact ties.
 * Replaces: the EPI_ARGMAX epilogue of the slot GEMM with its packed (score, ~row) key, model/kernels/decode.cu:90-96,
 * 189-230 (greedy slots). */
int nc_argmax_f32(const float *logits, int rows, int cols, long long ld, int32_t *out, void *stream);

/* Workspace bytes nc_choose_tokens needs for B slots over a vocabulary of `vocab` rows: per-workgroup keys. */
long long nc_choose_workspace_bytes(int B, int vocab);

/* Token choice and commit for every active slot b (active: [2][ceil(B / 64)] words, the active slots' bits, then
 * the masked slots'; slot b at bit b % 64 of word b / 64; NULL: every slot active, none masked). logits fp32
 * [B][ld], rows [0, vocab). A masked slot may choose only the rows whose bit r % 32 of word r / 32 of its row of
 * allow ([B][ceil(vocab / 32)]) is set. temperature[b] == 0 (or temperature NULL): the largest raw logit, lowest row
 * on ties; > 0: Gumbel-max sampling of softmax(z / T), z = softcap tanh(s / softcap) (softcap <= 0: z = s), noise
 * from Philox4x32-10 at (row, pos[b] - first[b]) keyed by seed[b] (first NULL: 0); top_p[b] < 1 (T > 0): nucleus
 * sampling over the smallest set of rows whose probabilities sum past top_p (vocab <= 131072). Writes tokens[b]
 * (-1: no allowed row), alt_tokens[b] (the best allowed row but `lazy`, -1 if none or for a nucleus slot) and
 * pos[b] += 1. Inactive slots are untouched. Calls in one stream may share the workspace (nc_choose_workspace_bytes).
 * Replaces: the CHOICE ARGMAX epilogue, k_nucleus and k_commit, model/kernels/decode.cu:98-105,170-230,360-404,
 * 676-689 (host rules: inference/decoder.py:28-40). */
int nc_choose_tokens(const float *logits, int B, int vocab, long long ld, const unsigned long long *active,
                     const uint32_t *allow, const float *temperature, const float *top_p,
                     const unsigned long long *seed, const int32_t *first, int32_t *pos, float softcap, int lazy,
                     int32_t *tokens, int32_t *alt_tokens, void *workspace, long long workspace_bytes, void *stream);

/* Residual add fused with the RMS norm over rows of d bf16 (contiguous, d % 8 == 0, d <= 8192): x_out = bf16(x +
 * delta) (delta NULL: x_out = x; x_out NULL: not stored; x_out may be x), y = bf16(x_out * r), r = 1 / sqrt(Σ
 * x_out² / d + FLT_EPSILON), Σ in fp32.
 * Replaces: the RESID epilogue of the slot GEMM and k_rstd, model/kernels/decode.cu:107-123,179-184,447-456; norm,
 * model/modeling.py:47-49. */
int nc_add_rms_norm_bf16(const void *x, const void *delta, void *x_out, void *y, int rows, int d, void *stream);

/* The value-embedding mix of a layer's projection rows, in place: per row r, n = bf16(x[r] rstd) (x: the layer
 * input, bf16 [rows][x_stride], d columns; the norm of nc_add_rms_norm_bf16), per kv head h
 * g = 2 sigmoid(gate[h] . n) (gate fp32 [hkv][d]), then v_h = bf16(v_h + g ve[tok[r]]_h) on the row's v heads
 * (qkv bf16 [rows][row_stride]: hq q heads, hkv k heads, hkv v heads; ve bf16 [vocab][hkv 128]). A row whose token
 * is outside [0, vocab) is left as is. d % 8 == 0, d <= 8192, hkv <= 64.
 * Replaces: the VE term of attn_prologue, model/kernels/decode.cu:476-493 (inference/modeling_nanochat.py:85-88). */
int nc_value_embed_bf16(void *qkv, long long row_stride, const void *x, long long x_stride, const int32_t *tok,
                        const void *ve, long long vocab, const float *gate, int rows, int d, int hq, int hkv,
                        void *stream);

/* out = bf16(relu(in)^2) over n bf16 (n % 8 == 0); out may be in.
 * Replaces: the RELU2 epilogue of the slot GEMM, model/kernels/decode.cu:174-178. */
int nc_relu2_bf16(const void *in, void *out, long long n, void *stream);

/* Epilogues of nc_slot_gemm_bf16 (s = Σ_k w[r][k] x[b][k] in fp32, rn = 1 / sqrt(Σ_k x[b][k]² / k + FLT_EPSILON)). */
enum {
    NC_GEMM_STORE = 0,      /* out bf16 = s */
    NC_GEMM_NORM_STORE = 1, /* out bf16 = s rn: the GEMM of the RMS-normed rows */
    NC_GEMM_RESID = 2,      /* out bf16 = bf16(s + res), one rounding; res may be out (in place) */
    NC_GEMM_RELU2_NORM = 3, /* out bf16 = relu(p) p, p = s rn */
    NC_GEMM_NORM_F32 = 4    /* out fp32 = s rn: logits */
};

/* The decode step's skinny weight GEMM: out[b][r] = epilogue(w[r] . x[b]) for b < m, r < n; w bf16 [n][k]
 * (nn.Linear layout), x bf16 [m][k], out [m][n] (bf16, fp32 for NORM_F32), all contiguous and 16-byte aligned;
 * n % 32 == 0, k % 64 == 0. Deterministic (fixed summation order). tile_n x tile_m picks the work tile (32 x 32,
 * 64 x 32, 32 x 64, 64 x 64, 32 x 128, 64 x 128, 128 x 64 or 128 x 128; n a multiple of tile_n); 0 x 0 chooses one
 * from the shape.
 * Replaces: the slot GEMM k_wgmma with its STORE / RESID / RELU2 epilogues and the rstd it applies (k_rstd),
 * model/kernels/decode.cu:107-123,169-184,292-338,447-456, launched per layer at :848-877. */
int nc_slot_gemm_bf16(const void *w, int n, int k, const void *x, int m, int epi, void *out, const void *res,
                      int tile_n, int tile_m, void *stream);

#ifdef __cplusplus
}
#endif

#endif
