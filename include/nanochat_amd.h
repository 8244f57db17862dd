/*
 * nanochat_amd: the C ABI of the MI355X (gfx950) fp8-KV decode path, libnanochat_amd.so.
 *
 * Conventions (the reference's, model/kernels/<name>.cu with native.py:43-65): every tensor is a raw device pointer,
 * counts are C ints, the HIP stream is the last argument, and every launch is stream-ordered and asynchronous.
 * Two error classes:
 *   - argument errors are checked on the host before any launch: the call returns a negative status and
 *     nc_last_error() names the problem (the reference validates in Python, inference/decoder.py:197-201);
 *   - a failed HIP runtime call or launch aborts the process with file:line (model/kernels/decode.cu:47-53).
 * Device-side, rows or keys whose position, sequence or block is out of range are skipped, never written or read
 * out of bounds.
 *
 * Cache layout (per layer), PAGE = 16 positions per block, D = 128: one pool, uint8 [num_blocks][Hkv][4224]; the
 * (block, kv head) tile is four 1 KiB parts of 64 16-byte fragments (a wave's MFMA operands in lane order), then
 * the scales:
 *   [0, 2048)     K codes: key t, dim d at ((d/16)%2)*1024 + (t + 16*(d/32))*16 + d%16
 *   [2048, 4096)  V codes, quad-transposed: key t, dim d at 2048 + ((d/4)%2)*1024 + (d/8 + 16*(t/4))*16 + (d%4)*4
 *                 + t%4
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

/* Position rows: positions [at, at + n) of sequence seq (any at, any n), every kv head, in `layers` pools spaced
 * pool_bytes apart (layer l's pool at cache + l * pool_bytes), to rows (uint8 [layers][n][hkv][264]: K codes
 * 128 B, V codes 128 B in dim order, K scale fp32, V scale fp32). A position whose block is missing gives a zero
 * row. Requires 0 <= seq < num_seqs, at + n <= max_blocks * 16.
 * Replaces: the device side of prompt_copy, model/kernels/decode.cu:1053-1075 (slot K/V rows to the prompt store,
 * position-granular bf16 rows there). */
int nc_kv_export_fp8(const uint8_t *cache, long long pool_bytes, int layers, const int32_t *block_table,
                     int max_blocks, int num_blocks, int num_seqs, int seq, int at, int n, int hkv, uint8_t *rows,
                     void *stream);

/* The inverse of nc_kv_export_fp8: rows (uint8 [layers][n][hkv][264]) into positions [at, at + n) of sequence seq;
 * only those positions' bytes of the pages change, and a position whose block is missing is not written.
 * Replaces: the load direction of prompt_copy, model/kernels/decode.cu:1053-1075. */
int nc_kv_import_fp8(const uint8_t *rows, int layers, uint8_t *cache, long long pool_bytes,
                     const int32_t *block_table, int max_blocks, int num_blocks, int num_seqs, int seq, int at, int n,
                     int hkv, void *stream);

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

/* nc_decode_step_fp8 with the sequence-local piece plan: every (sequence, kv head) segment of n pages (its keys'
 * pages) is cut into fixed pieces of max(piece_pages, ceil(n / P)) pages from its first page, P = the pieces
 * that cut the longest segment max_ctx admits into 16-page pieces (at least 32, at most 256), each piece's softmax
 * starts afresh, and the pieces merge in a fixed order set by the piece count; a wave takes whole pieces (the
 * balanced split's slice ends rounded to the nearest piece boundary). A sequence's output bits are then a function
 * of its own query, context and cache (and, for piece_pages below 16, of max_ctx) alone: decoded alone or in any
 * batch, it gets the same bits, as with the reference's one block per (head, slot). Arguments as
 * nc_decode_step_fp8, plus piece_pages in [1, 65536]; 16 measured fastest, and with 16 a segment's pieces are
 * max(16, ceil(n / 256)) pages whatever max_ctx is. The plain entry point's balanced split is 3 % faster on a
 * config-5 layer and 11 % on config 3's ragged batch, but its bits depend on the batch.
 * Replaces: k_prologue's append and k_attn (model/kernels/decode.cu:550-675), whose tokens depend on neither the
 * batch nor the store (inference/decoder.py:124-125); the decoder handle (dec_*) runs this entry point. */
int nc_decode_step_fp8_pieces(const void *qkv, long long row_stride, const int32_t *pos, int32_t *pos_out,
                              const float *q_gain, const float *k_gain, const float *cos, const float *sin,
                              int rope_len, uint8_t *cache, const int32_t *block_table, int max_blocks,
                              int num_blocks, int window, int B, int hq, int hkv, int max_ctx, float sm_scale,
                              int piece_pages, void *out, void *workspace, long long workspace_bytes, void *stream);

/* nc_decode_step_fp8 without the workspace: the partial results between its two kernels live in a static device
 * array of 64 MiB (67108864 bytes), a code object of its own that a device loads when this entry first runs on it
 * and holds until the process ends, so the call allocates nothing. A shape whose workspace (nc_decode_workspace_bytes) exceeds 64 MiB is rejected with an
 * error (config 3's B 64, 16 / 4 heads need 21.5 MB; B 128 of 13 MHA heads 11.9 MB). Every call on a device shares
 * its array: calls in one stream are ordered, calls that may overlap on one device (two streams) race. Outputs, cache
 * bytes and pos_out are bit-identical to nc_decode_step_fp8's.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). */
int nc_decode_step_fp8_noalloc(const void *qkv, long long row_stride, const int32_t *pos, int32_t *pos_out,
                               const float *q_gain, const float *k_gain, const float *cos, const float *sin,
                               int rope_len, uint8_t *cache, const int32_t *block_table, int max_blocks,
                               int num_blocks, int window, int B, int hq, int hkv, int max_ctx, float sm_scale,
                               void *out, void *stream);

/* Chunked-prefill attention: row r (bf16 q [n][Hq][128], normed and rotated, e.g. nc_kv_append_fp8's q_out) at
 * position pos[r] of sequence seq[r] attends keys [max(pos - window, 0), pos] of that sequence in the cache
 * (window < 0: all), query head h reading kv head h / (Hq / Hkv), scores times sm_scale, fp32 softmax, bf16 out
 * [n][Hq][128]. The rows' own keys must be in the cache already (append the whole chunk first), so each row sees
 * the chunk's earlier rows causally. Rows with pos < 0 or seq outside [0, num_seqs) get zero rows; a row's G
 * heads of one kv head whose q holds an infinity or a NaN (nc_kv_append_fp8's q rows past the rotary table) get
 * NaN rows, as the fused decode step does there, and change no other row. Keys of a missing block are skipped.
 * Rows may come in any order; a sequence's rows being consecutive is fastest.
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

/* The embedding and its norm: x[r] = bf16(e r) for e = table[tok[r]] (fp32 if table_fp32, else bf16; [vocab][d]),
 * r = 1 / sqrt(Σ e² / d + FLT_EPSILON), Σ in fp32 as nc_add_rms_norm_bf16 sums; x bf16 [rows][d]. A token outside
 * [0, vocab) gives a zero row. d % 8 == 0, d <= 8192.
 * Replaces: k_norm's EMBED kind, model/kernels/decode.cu:413-441 (x0 = norm(embed(tok)), kept fp32 there, bf16 here
 * as in inference/modeling_nanochat.py:150-165). */
int nc_embed_rms_norm(const void *table, int table_fp32, long long vocab, const int32_t *tok, int rows, int d,
                      void *x, void *stream);

/* The per-layer residual mix, in place over n bf16 (n % 8 == 0): x = bf16(lr x + l0 x0), products and sum in fp32.
 * Replaces: k_norm's RESID_NORM mix, model/kernels/decode.cu:428-431 (inference/modeling_nanochat.py:170-171). */
int nc_mix_bf16(void *x, const void *x0, long long n, float lr, float l0, void *stream);

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

/* nc_slot_gemm_bf16 whose launch also reads [prefetch, prefetch + prefetch_bytes) (16-byte aligned; whole 64 KiB
 * blocks, the rest is skipped) on the compute units the tiles leave idle, and discards it: bytes read so sit in the
 * memory-side cache for the next kernel. A decode step passes the next GEMM's weights (the up GEMM W_down, the down
 * GEMM the next layer's W_qkv, the qkv GEMM W_o), which the next GEMM then streams from that cache instead of HBM.
 * Outputs are bit-identical to nc_slot_gemm_bf16's; with the many-rows tile (m >= 512, tile 0 x 0) nothing is read.
 * No counterpart in the reference (its k_wgmma streams each layer's weights from HBM). */
int nc_slot_gemm_bf16_prefetch(const void *w, int n, int k, const void *x, int m, int epi, void *out, const void *res,
                               int tile_n, int tile_m, const void *prefetch, long long prefetch_bytes, void *stream);

/* ------------------------------------------------------------------------------------------------------------
 * The decoder handle (the reference's dec_* runtime, model/kernels/decode.cu:693-1131, bound by
 * inference/decoder.py:129-324): B slots of at most max_len positions over this library's kernels, an fp8 cache per
 * layer, captured step graphs over all slots and over the first 256, pinned token and mask buffers, and a prompt
 * store in pinned host memory. One host thread; every call is ordered on the handle's stream (the caller's, not the
 * legacy default stream, alive past dec_destroy); dec_tokens is the only call that waits. Weights are borrowed and
 * must stay unchanged while the handle lives. As the reference's handle (decode.cu:47-53,927-931), a call that cannot
 * do what it was asked (an argument out of range, a failed HIP call) prints a message and aborts; only
 * dec_create_v2, which the reference does not have, returns NULL with nc_last_error() instead.
 */

/* cfg: L, C (hidden size, a multiple of 128), F (MLP width, a multiple of 64), vocab (<= 131072), max_len (positions
 * per slot; cos / sin hold at least that many rows), store (prompt-store positions), lazy (the token whose
 * alternative each choice also reports, BOS). ptrs: wte (fp32 [vocab][C]), cos, sin (fp32 [max_len][64]), lm_head
 * (bf16 [vocab][C]), then per layer qkv ([(H + 2 Hkv) 128][C]), o, up ([F][C]), down ([C][F]) (bf16), the
 * value-embedding table (bf16 [vocab][Hkv 128]) and its gate (fp32 [Hkv][C]) or 0, 0, and the q and k norm gains
 * (fp32 [128]). scal: per layer the residual and x0 lambdas, then the logit cap. window: per layer, keys before a
 * query (< 0: all). Aborts with a message on a bad argument. H = C / 128; the slot count is the most whose caches
 * fit the free device memory, at most 1024.
 * Replaces: dec_create, model/kernels/decode.cu:950-1023 (same arguments; the cache is fp8). */
void *dec_create(const int *cfg, const uint64_t *ptrs, const float *scal, const int *window, void *stream);

/* dec_create with ncfg configuration fields: cfg[7] Hkv (0: H), cfg[8] the slot count (0: as dec_create),
 * cfg[9] 1 for a bf16 embedding table. Returns NULL on a bad argument (nc_last_error). No counterpart in the
 * reference: its fields 0-6 keep their meaning and the new ones are appended, as the grouped-query caches and bf16
 * checkpoint exports need. */
void *dec_create_v2(const int *cfg, int ncfg, const uint64_t *ptrs, const float *scal, const int *window,
                    void *stream);

/* Releases every resource of the handle (after waiting for its stream). Replaces: dec_destroy, decode.cu:904-924. */
void dec_destroy(void *handle);

/* The handle's slot count. Replaces: dec_batch, decode.cu:948. */
int dec_batch(void *handle);

/* Rows per dec_prefill call (16384; the reference's 1024: its caller chunks by this value). Replaces:
 * dec_prefill_rows, decode.cu:1037. */
int dec_prefill_rows(void *handle);

/* Slot b starts at its prompt's last token `token`, position `last` (earlier positions cached or queued for
 * prefill), with its sampling parameters (inference/decoder.py:28-40). Replaces: dec_set_prompt, decode.cu:1026-1035. */
void dec_set_prompt(void *handle, int b, int32_t token, int32_t last, float temperature, float top_p,
                    unsigned long long seed);

/* Runs n <= dec_prefill_rows rows (rows: int32 [3][n], tokens, positions, slots) through every layer, caching each
 * row's key and value; a row attends its slot's cached positions and the earlier rows of the call. Stream-ordered:
 * rows is copied into one of a ring of pinned staging buffers before the call returns (the host waits only when
 * that buffer's copy from 4 calls earlier is still pending). Replaces: dec_prefill, decode.cu:1041-1051. */
void dec_prefill(void *handle, int n, const int32_t *rows);

/* Slot b's cache positions [at, at + n), every layer, to the prompt store's positions [store_at, store_at + n)
 * (save) or back (load); any positions (the store holds nc_kv_export_fp8 rows, [L][store][Hkv][264]). Stream-ordered.
 * A slot, range or store position out of bounds aborts with a message, as every other failure of the handle.
 * Replaces: dec_save_prompt / dec_load_prompt, decode.cu:1069-1075 (bf16 rows there). */
void dec_save_prompt(void *handle, int b, int at, int store_at, int n);
void dec_load_prompt(void *handle, int b, int at, int store_at, int n);

/* The pinned allowed-token rows [B][ceil(vocab / 32)] (bit t % 32 of word t / 32 of row b: slot b may choose t),
 * written by the caller between dec_tokens and dec_set_active. Replaces: dec_masks, decode.cu:1079. */
uint32_t *dec_masks(void *handle);

/* The active and masked slots, slots[2][ceil(B / 64)] (slot b at bit b % 64 of word b / 64); the masked slots'
 * rows of dec_masks are copied; a slot that is not active idles (position -1). The next launches run the narrow
 * graphs when no slot past the first 256 is active. Replaces: dec_set_active, decode.cu:1083-1105. */
void dec_set_active(void *handle, const unsigned long long *slots);

/* Launch a step's body (embedding, every layer) and its head (lm_head, the choice and its commit: each active slot's
 * next token, position + 1). Replaces: dec_launch_body / dec_launch_head, decode.cu:1107-1116. */
void dec_launch_body(void *handle);
void dec_launch_head(void *handle);

/* Waits for the launched step; out[b]: the token slot b took, out[B + b]: its alternative, the best allowed token
 * but lazy (-1 if none; stale for idle slots). Replaces: dec_tokens, decode.cu:1120-1124. */
void dec_tokens(void *handle, int32_t *out);

/* Slot b's next input becomes its last alternative (the host rejected the lazy token). Replaces: dec_take_alt,
 * decode.cu:1128-1131. */
void dec_take_alt(void *handle, int b);

#ifdef __cplusplus
}
#endif

#endif
