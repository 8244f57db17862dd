/*
 * The decoder handle: the reference's native decode runtime (the Decoder of model/kernels/decode.cu:693-1131, bound
 * by inference/decoder.py:129-324 through the dec_* functions) rebuilt over this library's kernels, with the same
 * entry points and calling protocol.
 *
 * A handle holds B slots of at most max_len positions:
 *   - per layer a contiguous fp8 cache pool (slot b's pages are blocks b * max_blocks + i, nc_kv_append_fp8's
 *     layout), zeroed at creation;
 *   - the activations of B decode rows and of DEC_ROWS prefill rows;
 *   - the slot state on the device: next input token, position (-1: idle), first generated position, temperature,
 *     top_p, seed, the active / masked slot words and the allowed-token rows;
 *   - two captured hipGraphs per width, the body (embedding, norm, every layer) and the head (lm_head and the token
 *     choice with its commit), over all B slots and, when B > DEC_NARROW, over the first DEC_NARROW slots (the
 *     reference's narrow graphs, decode.cu:995-1005);
 *   - pinned host memory for the tokens, the allowed-token rows (dec_masks), a ring of DEC_STAGES prefill row
 *     buffers and the prompt store, and a device staging buffer for the store's copies.
 *
 * The prompt store holds positions as nc_kv_export_fp8 rows, [L][store][Hkv][264] (a position's K and V codes
 * and scales), so dec_save_prompt / dec_load_prompt move any positions of a slot to any store positions: a kernel
 * packs the slot's pages into the staging rows and one 2-D copy moves them (L rows of n positions) to the store, or
 * the reverse. Everything is ordered on the handle's stream.
 *
 * A decode step is dec_set_active, dec_launch_body, dec_launch_head, dec_tokens. The body runs per layer: the
 * residual mix (nc_mix_bf16, where it is not the identity), the qkv slot GEMM of the normed rows, the
 * value-embedding mix (nc_value_embed_bf16), the fused append + attention (nc_decode_step_fp8_pieces: sequence-local
 * pieces, so a request's bits do not depend on the batch), the o projection (RESID), up (RELU2_NORM) and down
 * (RESID) GEMMs. The head is the lm_head GEMM (NORM_F32) and nc_choose_tokens,
 * which writes each active slot's choice as its next input token and advances its position (k_commit). Idle slots
 * carry position -1: the decode step does no work for them and the choice leaves them untouched.
 *
 * Small host-to-device updates (a slot's prompt state, the slot words, dec_take_alt) are kernels whose values travel
 * in the kernel arguments, so no host buffer is read after the call returns. dec_prefill's rows (up to 192 KB) go
 * through the ring of pinned buffers, each guarded by an event recorded after its copy.
 *
 * Errors follow the reference's handle (decode.cu:47-53,927-931): an argument out of range or a failed HIP call
 * prints a message and aborts, so a caller that ignores return values never decodes from a cache it did not get.
 * dec_create_v2 alone returns NULL (with nc_last_error) on a bad configuration.
 */
#include <string.h>

#include "layout.h"
#include "nanochat_amd.h"

#define DEC_MAX_BATCH 1024 /* slots at most (decode.cu:28-29) */
#define DEC_NARROW 256     /* the narrow graphs' slots (decode.cu:32-33) */
#define DEC_ROWS 16384     /* prefill rows per dec_prefill (the reference runs 1024, decode.cu:1037; its caller chunks by
                              dec_prefill_rows, so more rows a call keep the GEMMs on their many-rows tile) */
#define DEC_STAGES 4       /* pinned staging buffers of prefill rows in flight */
#define DEC_ROW_BYTES 264  /* one position of one kv head in the prompt store (nc_kv_export_fp8's rows) */
#define DEC_WORDS (DEC_MAX_BATCH / 64)
#define DEC_GLOBAL_PTRS 4
#define DEC_LAYER_PTRS 8
#define DEC_SM_SCALE 0.08838834764831845f /* 1 / sqrt(128) */
/* The decode attention's sequence-local pieces (nc_decode_step_fp8_pieces): a request's tokens depend on neither the
 * batch nor the store, as the reference promises (inference/decoder.py:124-125). */
#define DEC_PIECE_PAGES 16

struct DecLayer {
    const void *qkv, *o, *up, *down, *ve; /* bf16 weights [out][in]; ve [vocab][Hkv 128] or null */
    const float *ve_gate, *q_gain, *k_gain;
    float lr, l0; /* the residual mix: bf16(lr x + l0 x0) */
    int window;
};

/* Activations of up to `cap` rows. */
struct DecRows {
    int32_t *tok, *pos, *seq;
    bf16_t *x, *x0, *qkv, *q, *o, *u;
    float *logits;
};

struct Decoder {
    int L, C, F, vocab, vocab_pad, max_len, store_len, lazy, H, Hkv, B, max_blocks, wte_fp32, mixes, words;
    float softcap;
    const void *wte, *lm_head;
    const float *cos, *sin;
    void *lm_pad; /* lm_head with zero rows up to a multiple of 32, when the vocabulary is not one */
    DecLayer *layer;
    hipStream_t stream;
    uint8_t *cache;
    size_t pool_bytes; /* one layer's pool */
    DecRows d, r;      /* decode rows (B), prefill rows (DEC_ROWS) */
    int32_t *first, *alt;
    float *temperature, *top_p;
    unsigned long long *seed;
    unsigned long long *slots[2]; /* [2][words], full and narrow */
    uint32_t *allow;              /* [B][vocab / 32] */
    void *ws_dec, *ws_choose;
    long long ws_dec_bytes, ws_choose_bytes;
    int32_t *host_tokens, *host_rows; /* host_rows: pinned [DEC_STAGES][3][DEC_ROWS] */
    hipEvent_t staged[DEC_STAGES];    /* recorded after the copy out of host_rows' stage */
    int stage;                        /* the next stage dec_prefill fills */
    uint32_t *host_allow;
    uint8_t *store;   /* pinned [L][store][Hkv][264] */
    uint8_t *staging; /* device [L][max_len][Hkv][264]: a prompt's rows between the slot and the store */
    int narrow;     /* the next launches use the narrow graphs */
    hipGraphExec_t body[2], head[2];
    void *blocks[32]; /* device allocations, freed by dec_destroy */
    int nblocks;
};

static void *dec_alloc(Decoder *d, size_t bytes) {
    if (d->nblocks == (int)(sizeof d->blocks / sizeof d->blocks[0])) {
        fprintf(stderr, "decoder.hip: more device blocks than the handle records\n");
        abort();
    }
    void *p = nullptr;
    NC_HIP_CHECK(hipMalloc(&p, bytes < 256 ? 256 : bytes));
    NC_HIP_CHECK(hipMemsetAsync(p, 0, bytes < 256 ? 256 : bytes, d->stream));
    d->blocks[d->nblocks++] = p;
    return p;
}

static void rows_alloc(Decoder *d, DecRows &r, int cap, bool logits) {
    const size_t C = d->C, qkv = (size_t)(d->H + 2 * d->Hkv) * NC_HEAD_DIM, hd = (size_t)d->H * NC_HEAD_DIM;
    r.tok = (int32_t *)dec_alloc(d, 3 * (size_t)cap * sizeof(int32_t));
    r.pos = r.tok + cap;
    r.seq = r.tok + 2 * cap;
    r.x = (bf16_t *)dec_alloc(d, cap * C * 2);
    r.x0 = d->mixes ? (bf16_t *)dec_alloc(d, cap * C * 2) : nullptr;
    r.qkv = (bf16_t *)dec_alloc(d, cap * qkv * 2);
    r.q = (bf16_t *)dec_alloc(d, cap * hd * 2);
    r.o = (bf16_t *)dec_alloc(d, cap * hd * 2);
    r.u = (bf16_t *)dec_alloc(d, cap * (size_t)d->F * 2);
    r.logits = logits ? (float *)dec_alloc(d, cap * (size_t)d->vocab_pad * sizeof(float)) : nullptr;
}

static uint8_t *pool(const Decoder *d, int l) { return d->cache + (size_t)l * d->pool_bytes; }

#define DEC_TRY(call)              \
    do {                           \
        const int rc_ = (call);    \
        if (rc_ < 0) return rc_;   \
    } while (0)

/* Embedding, norm and the x0 copy of n rows. */
static int enqueue_embed(Decoder *d, DecRows &r, int n) {
    DEC_TRY(nc_embed_rms_norm(d->wte, d->wte_fp32, d->vocab, r.tok, n, d->C, r.x, d->stream));
    if (d->mixes)
        NC_HIP_CHECK(hipMemcpyAsync(r.x0, r.x, (size_t)n * d->C * 2, hipMemcpyDeviceToDevice, d->stream));
    return 0;
}

/* The part of layer l before attention: mix, qkv GEMM of the normed rows, value-embedding mix. */
static int enqueue_qkv(Decoder *d, DecRows &r, int n, int l) {
    const DecLayer &ly = d->layer[l];
    const int cols = (d->H + 2 * d->Hkv) * NC_HEAD_DIM;
    if (d->mixes && (ly.lr != 1.0f || ly.l0 != 0.0f))
        DEC_TRY(nc_mix_bf16(r.x, r.x0, (long long)n * d->C, ly.lr, ly.l0, d->stream));
    /* each decode GEMM's idle compute units pull the next GEMM's weights into the memory-side cache (here W_o;
     * the many-rows tile of a long prefill reads nothing extra) */
    DEC_TRY(nc_slot_gemm_bf16_prefetch(ly.qkv, cols, d->C, r.x, n, NC_GEMM_NORM_STORE, r.qkv, nullptr, 0, 0, ly.o,
                                       (long long)d->C * d->H * NC_HEAD_DIM * 2, d->stream));
    if (ly.ve)
        DEC_TRY(nc_value_embed_bf16(r.qkv, cols, r.x, d->C, r.tok, ly.ve, d->vocab, ly.ve_gate, n, d->C, d->H, d->Hkv,
                                    d->stream));
    return 0;
}

/* The part of layer l after attention (o in r.o): x += o_proj(o); x += down(relu(up(norm(x)))^2). */
static int enqueue_mlp(Decoder *d, DecRows &r, int n, int l) {
    const DecLayer &ly = d->layer[l];
    const int hd = d->H * NC_HEAD_DIM;
    /* the up GEMM pulls W_down, the down GEMM the next layer's W_qkv (the o GEMM is too short to hide W_up's read) */
    const void *next_qkv = l + 1 < d->L ? d->layer[l + 1].qkv : nullptr;
    const long long qkv_bytes = next_qkv ? (long long)(d->H + 2 * d->Hkv) * NC_HEAD_DIM * d->C * 2 : 0;
    DEC_TRY(nc_slot_gemm_bf16(ly.o, d->C, hd, r.o, n, NC_GEMM_RESID, r.x, r.x, 0, 0, d->stream));
    DEC_TRY(nc_slot_gemm_bf16_prefetch(ly.up, d->F, d->C, r.x, n, NC_GEMM_RELU2_NORM, r.u, nullptr, 0, 0, ly.down,
                                       (long long)d->C * d->F * 2, d->stream));
    DEC_TRY(nc_slot_gemm_bf16_prefetch(ly.down, d->C, d->F, r.u, n, NC_GEMM_RESID, r.x, r.x, 0, 0, next_qkv, qkv_bytes,
                                       d->stream));
    return 0;
}

/* A decode step's body over slots [0, n). */
static int enqueue_body(Decoder *d, int n) {
    DecRows &r = d->d;
    const int cols = (d->H + 2 * d->Hkv) * NC_HEAD_DIM;
    DEC_TRY(enqueue_embed(d, r, n));
    for (int l = 0; l < d->L; l++) {
        const DecLayer &ly = d->layer[l];
        DEC_TRY(enqueue_qkv(d, r, n, l));
        DEC_TRY(nc_decode_step_fp8_pieces(r.qkv, cols, r.pos, nullptr, ly.q_gain, ly.k_gain, d->cos, d->sin,
                                          d->max_len, pool(d, l), nullptr, d->max_blocks, d->B * d->max_blocks,
                                          ly.window, n, d->H, d->Hkv, d->max_len, DEC_SM_SCALE, DEC_PIECE_PAGES, r.o,
                                          d->ws_dec, d->ws_dec_bytes, d->stream));
        DEC_TRY(enqueue_mlp(d, r, n, l));
    }
    return 0;
}

/* A decode step's head over slots [0, n): logits, the choice into each active slot's next token, the commit. */
static int enqueue_head(Decoder *d, int n, int narrow) {
    DecRows &r = d->d;
    const void *lm = d->lm_pad ? d->lm_pad : d->lm_head;
    DEC_TRY(nc_slot_gemm_bf16(lm, d->vocab_pad, d->C, r.x, n, NC_GEMM_NORM_F32, r.logits, nullptr, 0, 0, d->stream));
    DEC_TRY(nc_choose_tokens(r.logits, n, d->vocab, d->vocab_pad, d->slots[narrow], d->allow, d->temperature,
                             d->top_p, d->seed, d->first, r.pos, d->softcap, d->lazy, r.tok, d->alt, d->ws_choose,
                             d->ws_choose_bytes, d->stream));
    return 0;
}

/* Prefill rows [0, n) of d->r: every row's key and value cached before any row attends (decode.cu:859-863); the
 * last layer stops after its append (no row chooses a token). */
static int enqueue_prefill(Decoder *d, int n) {
    DecRows &r = d->r;
    const int cols = (d->H + 2 * d->Hkv) * NC_HEAD_DIM;
    DEC_TRY(enqueue_embed(d, r, n));
    for (int l = 0; l < d->L; l++) {
        const DecLayer &ly = d->layer[l];
        DEC_TRY(enqueue_qkv(d, r, n, l));
        DEC_TRY(nc_kv_append_fp8(r.qkv, cols, n, r.pos, r.seq, ly.q_gain, ly.k_gain, d->cos, d->sin, d->max_len, d->H,
                                 d->Hkv, r.q, pool(d, l), nullptr, d->max_blocks, d->B * d->max_blocks, d->B, nullptr,
                                 d->stream));
        if (l == d->L - 1) break;
        DEC_TRY(nc_prefill_attn_fp8(r.q, r.pos, r.seq, n, pool(d, l), nullptr, d->max_blocks, d->B * d->max_blocks,
                                    d->B, ly.window, d->H, d->Hkv, DEC_SM_SCALE, r.o, d->stream));
        DEC_TRY(enqueue_mlp(d, r, n, l));
    }
    return 0;
}

__global__ void k_set_slot(int32_t *tok, int32_t *pos, int32_t *first, float *temperature, float *top_p,
                           unsigned long long *seed, int b, int32_t token, int32_t last, float t, float p,
                           unsigned long long s) {
    tok[b] = token;
    pos[b] = last;
    first[b] = last;
    temperature[b] = t;
    top_p[b] = p;
    seed[b] = s;
}

struct DecWords {
    unsigned long long w[2 * DEC_WORDS];
};

/* The slot words of both widths (full [2][words], narrow [2][DEC_NARROW / 64]: the first words of each row), and
 * position -1 for every slot that is not active, so the body does no work for it. */
__global__ void k_set_words(DecWords in, int words, unsigned long long *full, unsigned long long *narrow,
                            int32_t *pos, int B) {
    const int i = threadIdx.x;
    if (i < 2 * words) full[i] = in.w[i];
    if (narrow && i < 2 * (DEC_NARROW / 64)) {
        const int row = i / (DEC_NARROW / 64), k = i % (DEC_NARROW / 64);
        narrow[i] = in.w[row * words + k];
    }
    for (int b = i; b < B; b += blockDim.x)
        if (!((in.w[b / 64] >> (b % 64)) & 1ull)) pos[b] = -1;
}

__global__ void k_take_alt(int32_t *tok, const int32_t *alt, int b) { tok[b] = alt[b]; }

static hipGraphExec_t capture(Decoder *d, int n, int narrow, bool head, int *rc) {
    hipGraph_t graph;
    hipGraphExec_t exec = nullptr;
    NC_HIP_CHECK(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
    *rc = head ? enqueue_head(d, n, narrow) : enqueue_body(d, n);
    NC_HIP_CHECK(hipStreamEndCapture(d->stream, &graph));
    if (*rc == 0) NC_HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    NC_HIP_CHECK(hipGraphDestroy(graph));
    return exec;
}

/* Teardown never aborts (it may run from a finalizer late in a process): failures are ignored; hipFree waits for
 * the device. */
extern "C" void dec_destroy(void *handle) {
    Decoder *d = (Decoder *)handle;
    if (!d) return;
    for (int i = 0; i < 2; i++) {
        if (d->body[i]) (void)hipGraphExecDestroy(d->body[i]);
        if (d->head[i]) (void)hipGraphExecDestroy(d->head[i]);
    }
    for (int i = 0; i < DEC_STAGES; i++)
        if (d->staged[i]) (void)hipEventDestroy(d->staged[i]);
    for (int i = 0; i < d->nblocks; i++) (void)hipFree(d->blocks[i]);
    for (void *p : {(void *)d->host_tokens, (void *)d->host_rows, (void *)d->host_allow, (void *)d->store})
        if (p) (void)hipHostFree(p);
    free(d->layer);
    free(d);
}

/* Bytes of one slot's cache over every layer. */
static size_t slot_bytes(int L, int max_blocks, int hkv) { return (size_t)L * max_blocks * hkv * NC_TILE_BYTES; }

static int create(Decoder *d, const int *cfg, int ncfg, const uint64_t *ptrs, const float *scal, const int *window) {
    NC_REQUIRE(cfg && ptrs && scal && window, "dec_create: null argument");
    NC_REQUIRE(ncfg >= 7, "dec_create_v2: %d config fields, at least 7", ncfg);
    d->L = cfg[0]; d->C = cfg[1]; d->F = cfg[2]; d->vocab = cfg[3]; d->max_len = cfg[4];
    d->lazy = cfg[6];
    d->H = d->C / NC_HEAD_DIM;
    d->Hkv = ncfg > 7 && cfg[7] > 0 ? cfg[7] : d->H;
    const int batch = ncfg > 8 ? cfg[8] : 0;
    d->wte_fp32 = ncfg > 9 ? cfg[9] == 0 : 1; /* field 9: 1 for a bf16 embedding table; the reference's is fp32 */
    NC_REQUIRE(d->L > 0 && d->C > 0 && d->C % NC_HEAD_DIM == 0 && d->C <= 8192,
               "dec_create: L %d, C %d (a multiple of 128, at most 8192)", d->L, d->C);
    NC_REQUIRE(d->F > 0 && d->F % 64 == 0, "dec_create: F %d must be a multiple of 64", d->F);
    NC_REQUIRE(d->vocab > 0 && d->vocab <= 131072, "dec_create: vocab %d outside [1, 131072]", d->vocab);
    NC_REQUIRE(d->max_len > 0, "dec_create: max_len %d", d->max_len);
    NC_REQUIRE(d->Hkv > 0 && d->H % d->Hkv == 0 && d->H / d->Hkv <= 16, "dec_create: %d heads over %d kv heads", d->H,
               d->Hkv);
    NC_REQUIRE(cfg[5] >= 0 && batch >= 0 && batch <= DEC_MAX_BATCH, "dec_create: store %d, batch %d", cfg[5], batch);
    d->max_blocks = (d->max_len + NC_PAGE - 1) / NC_PAGE;
    d->store_len = cfg[5]; /* prompt-store positions */
    d->vocab_pad = (d->vocab + 31) / 32 * 32;
    d->wte = (const void *)ptrs[0];
    d->cos = (const float *)ptrs[1];
    d->sin = (const float *)ptrs[2];
    d->lm_head = (const void *)ptrs[3];
    NC_REQUIRE(d->wte && d->cos && d->sin && d->lm_head, "dec_create: null global weight");
    d->softcap = scal[2 * d->L];
    d->layer = (DecLayer *)calloc(d->L, sizeof(DecLayer));
    for (int l = 0; l < d->L; l++) {
        const uint64_t *p = ptrs + DEC_GLOBAL_PTRS + DEC_LAYER_PTRS * l;
        d->layer[l] = {(const void *)p[0], (const void *)p[1], (const void *)p[2], (const void *)p[3],
                       (const void *)p[4], (const float *)p[5], (const float *)p[6], (const float *)p[7], scal[2 * l],
                       scal[2 * l + 1], window[l]};
        const DecLayer &ly = d->layer[l];
        NC_REQUIRE(ly.qkv && ly.o && ly.up && ly.down && ly.q_gain && ly.k_gain && (!ly.ve || ly.ve_gate),
                   "dec_create: layer %d: null weight", l);
        if (ly.lr != 1.0f || ly.l0 != 0.0f) d->mixes = 1;
    }
    const size_t per_slot = slot_bytes(d->L, d->max_blocks, d->Hkv);
    if (batch > 0) {
        d->B = batch;
    } else { /* the most slots whose caches fit the free memory, keeping 1 GiB and a tenth for the rest */
        size_t free_bytes = 0, total_bytes = 0;
        NC_HIP_CHECK(hipMemGetInfo(&free_bytes, &total_bytes));
        const size_t room = free_bytes > (1ull << 30) ? (free_bytes - (1ull << 30)) / 10 * 9 : 0;
        d->B = (int)(room / per_slot < DEC_MAX_BATCH ? room / per_slot : DEC_MAX_BATCH);
        NC_REQUIRE(d->B > 0, "dec_create: no slot of %zu bytes fits the free device memory", per_slot);
    }
    d->words = (d->B + 63) / 64;
    d->pool_bytes = (size_t)d->B * d->max_blocks * d->Hkv * NC_TILE_BYTES;
    d->cache = (uint8_t *)dec_alloc(d, d->pool_bytes * d->L);
    rows_alloc(d, d->d, d->B, true);
    rows_alloc(d, d->r, DEC_ROWS, false);
    d->first = (int32_t *)dec_alloc(d, 2 * (size_t)d->B * sizeof(int32_t));
    d->alt = d->first + d->B;
    d->temperature = (float *)dec_alloc(d, 2 * (size_t)d->B * sizeof(float));
    d->top_p = d->temperature + d->B;
    d->seed = (unsigned long long *)dec_alloc(d, (size_t)d->B * 8);
    d->slots[0] = (unsigned long long *)dec_alloc(d, 2 * (size_t)d->words * 8);
    d->slots[1] = d->B > DEC_NARROW ? (unsigned long long *)dec_alloc(d, 2 * (DEC_NARROW / 64) * 8) : nullptr;
    const size_t allow_words = (size_t)(d->vocab + 31) / 32;
    d->allow = (uint32_t *)dec_alloc(d, (size_t)d->B * allow_words * 4);
    d->ws_dec_bytes = nc_decode_workspace_bytes(d->B, d->H, d->Hkv, d->max_len);
    d->ws_dec = dec_alloc(d, d->ws_dec_bytes);
    d->ws_choose_bytes = nc_choose_workspace_bytes(d->B, d->vocab);
    d->ws_choose = dec_alloc(d, d->ws_choose_bytes);
    if (d->vocab_pad != d->vocab) { /* zero rows past the vocabulary: their logits are never chosen */
        d->lm_pad = dec_alloc(d, (size_t)d->vocab_pad * d->C * 2);
        NC_HIP_CHECK(hipMemcpyAsync(d->lm_pad, d->lm_head, (size_t)d->vocab * d->C * 2, hipMemcpyDeviceToDevice,
                                    d->stream));
    }
    NC_HIP_CHECK(hipMemsetD32Async((hipDeviceptr_t)d->d.pos, -1, d->B, d->stream)); /* every slot idle */
    NC_HIP_CHECK(hipMemsetD32Async((hipDeviceptr_t)d->top_p, 0x3f800000, d->B, d->stream)); /* top_p 1 */
    NC_HIP_CHECK(hipHostMalloc((void **)&d->host_tokens, 2 * (size_t)d->B * sizeof(int32_t), hipHostMallocDefault));
    NC_HIP_CHECK(hipHostMalloc((void **)&d->host_rows, DEC_STAGES * 3 * (size_t)DEC_ROWS * sizeof(int32_t),
                               hipHostMallocDefault));
    for (int i = 0; i < DEC_STAGES; i++) { /* recorded once, so the first wait on each stage returns at once */
        NC_HIP_CHECK(hipEventCreateWithFlags(&d->staged[i], hipEventDisableTiming));
        NC_HIP_CHECK(hipEventRecord(d->staged[i], d->stream));
    }
    NC_HIP_CHECK(hipHostMalloc((void **)&d->host_allow, (size_t)d->B * allow_words * 4, hipHostMallocDefault));
    memset(d->host_allow, 0, (size_t)d->B * allow_words * 4);
    if (d->store_len) {
        const size_t position = (size_t)d->L * d->Hkv * DEC_ROW_BYTES;
        NC_HIP_CHECK(hipHostMalloc((void **)&d->store, position * d->store_len, hipHostMallocDefault));
        d->staging = (uint8_t *)dec_alloc(d, position * d->max_len);
    }
    /* every launch path once eagerly (no slot active: nothing is written but scratch rows), then the graphs */
    const int widths[2] = {d->B, d->B > DEC_NARROW ? DEC_NARROW : 0};
    for (int g = 0; g < 2; g++) {
        if (!widths[g]) continue;
        DEC_TRY(enqueue_body(d, widths[g]));
        DEC_TRY(enqueue_head(d, widths[g], g));
    }
    NC_HIP_CHECK(hipStreamSynchronize(d->stream));
    for (int g = 0; g < 2; g++) {
        if (!widths[g]) continue;
        int rc = 0;
        d->body[g] = capture(d, widths[g], g, false, &rc);
        DEC_TRY(rc);
        d->head[g] = capture(d, widths[g], g, true, &rc);
        DEC_TRY(rc);
    }
    return 0;
}

/* cfg: L, C, F, vocab, max_len (positions per slot), store (prompt-store positions), lazy (the token whose
 * alternative the choice also reports: BOS), then optionally Hkv (0: C / 128), batch (0: as many as fit, at most
 * 1024), embedding dtype (1: bf16; 0 or absent: fp32 as the reference's). */
extern "C" void *dec_create_v2(const int *cfg, int ncfg, const uint64_t *ptrs, const float *scal, const int *window,
                               void *stream) {
    Decoder *d = (Decoder *)calloc(1, sizeof(Decoder));
    d->stream = (hipStream_t)stream;
    if (create(d, cfg, ncfg, ptrs, scal, window) < 0) {
        char msg[512];
        strncpy(msg, nc_last_error(), sizeof msg - 1);
        msg[sizeof msg - 1] = 0;
        dec_destroy(d);
        nc_fail("%s", msg);
        return nullptr;
    }
    return d;
}

/* The reference's entry point aborts where dec_create_v2 returns NULL: its caller does not check the handle. */
extern "C" void *dec_create(const int *cfg, const uint64_t *ptrs, const float *scal, const int *window, void *stream) {
    void *h = dec_create_v2(cfg, 7, ptrs, scal, window, stream);
    if (!h) {
        fprintf(stderr, "dec_create: %s\n", nc_last_error());
        abort();
    }
    return h;
}

extern "C" int dec_batch(void *handle) { return ((Decoder *)handle)->B; }

extern "C" int dec_prefill_rows(void *) { return DEC_ROWS; }

extern "C" uint32_t *dec_masks(void *handle) { return ((Decoder *)handle)->host_allow; }

extern "C" void dec_set_prompt(void *handle, int b, int32_t token, int32_t last, float temperature, float top_p,
                               unsigned long long seed) {
    Decoder *d = (Decoder *)handle;
    if (b < 0 || b >= d->B) {
        fprintf(stderr, "dec_set_prompt: slot %d outside [0, %d)\n", b, d->B);
        abort();
    }
    hipLaunchKernelGGL(k_set_slot, dim3(1), dim3(1), 0, d->stream, d->d.tok, d->d.pos, d->first, d->temperature,
                       d->top_p, d->seed, b, token, last, temperature, top_p, seed);
    NC_LAUNCH_CHECK();
}

extern "C" void dec_prefill(void *handle, int n, const int32_t *rows) {
    Decoder *d = (Decoder *)handle;
    if (n <= 0) return;
    if (n > DEC_ROWS) {
        fprintf(stderr, "dec_prefill: %d rows exceed %d\n", n, DEC_ROWS);
        abort();
    }
    /* the stage's previous copy (DEC_STAGES calls ago) has read its buffer: usually long done, so no wait */
    const int k = d->stage;
    d->stage = (k + 1) % DEC_STAGES;
    NC_HIP_CHECK(hipEventSynchronize(d->staged[k]));
    int32_t *host = d->host_rows + (size_t)k * 3 * DEC_ROWS;
    for (int c = 0; c < 3; c++) memcpy(host + c * DEC_ROWS, rows + (size_t)c * n, n * sizeof(int32_t));
    const size_t pitch = (size_t)DEC_ROWS * sizeof(int32_t); /* the n rows of each of the 3 fields */
    NC_HIP_CHECK(hipMemcpy2DAsync(d->r.tok, pitch, host, pitch, n * sizeof(int32_t), 3, hipMemcpyHostToDevice,
                                  d->stream));
    NC_HIP_CHECK(hipEventRecord(d->staged[k], d->stream));
    if (enqueue_prefill(d, n) < 0) {
        fprintf(stderr, "dec_prefill: %s\n", nc_last_error());
        abort();
    }
}

/* Slot b's positions [at, at + n), every layer, to or from the store's positions [store_at, store_at + n): the
 * slot's pages <-> the staging rows by nc_kv_export_fp8 / nc_kv_import_fp8, the staging rows <-> the store by one
 * 2-D copy (L rows of n positions; the store's pitch is its whole layer). Out-of-range arguments abort. */
static void prompt_copy(Decoder *d, const char *name, int b, int at, int store_at, int n, bool to_store) {
    if (b < 0 || b >= d->B || at < 0 || n < 0 || store_at < 0 || (long long)at + n > d->max_len ||
        (long long)store_at + n > d->store_len) {
        fprintf(stderr, "%s: slot %d (of %d), positions [%d, %lld) (of %d), store positions [%d, %lld) (of %d)\n",
                name, b, d->B, at, (long long)at + n, d->max_len, store_at, (long long)store_at + n, d->store_len);
        abort();
    }
    if (n == 0) return;
    const size_t position = (size_t)d->Hkv * DEC_ROW_BYTES, width = (size_t)n * position;
    uint8_t *store = d->store + (size_t)store_at * position;
    const size_t store_pitch = (size_t)d->store_len * position;
    const int num_blocks = d->B * d->max_blocks;
    int rc = 0;
    if (to_store) {
        rc = nc_kv_export_fp8(d->cache, (long long)d->pool_bytes, d->L, nullptr, d->max_blocks, num_blocks, d->B, b,
                              at, n, d->Hkv, d->staging, d->stream);
        if (rc == 0)
            NC_HIP_CHECK(hipMemcpy2DAsync(store, store_pitch, d->staging, width, width, d->L, hipMemcpyDeviceToHost,
                                          d->stream));
    } else {
        NC_HIP_CHECK(hipMemcpy2DAsync(d->staging, width, store, store_pitch, width, d->L, hipMemcpyHostToDevice,
                                      d->stream));
        rc = nc_kv_import_fp8(d->staging, d->L, d->cache, (long long)d->pool_bytes, nullptr, d->max_blocks, num_blocks,
                              d->B, b, at, n, d->Hkv, d->stream);
    }
    if (rc < 0) {
        fprintf(stderr, "%s: %s\n", name, nc_last_error());
        abort();
    }
}

extern "C" void dec_save_prompt(void *handle, int b, int at, int store_at, int n) {
    prompt_copy((Decoder *)handle, "dec_save_prompt", b, at, store_at, n, true);
}

extern "C" void dec_load_prompt(void *handle, int b, int at, int store_at, int n) {
    prompt_copy((Decoder *)handle, "dec_load_prompt", b, at, store_at, n, false);
}

extern "C" void dec_set_active(void *handle, const unsigned long long *slots) {
    Decoder *d = (Decoder *)handle;
    DecWords w = {};
    memcpy(w.w, slots, 2 * (size_t)d->words * sizeof(unsigned long long));
    int high = -1, lo = -1, hi = -1;
    for (int i = 0; i < d->words; i++) {
        if (w.w[i]) high = i * 64 + 63 - __builtin_clzll(w.w[i]);
        const unsigned long long m = w.w[d->words + i];
        if (m) {
            if (lo < 0) lo = i * 64 + __builtin_ctzll(m);
            hi = i * 64 + 63 - __builtin_clzll(m);
        }
    }
    d->narrow = d->body[1] && high < DEC_NARROW;
    hipLaunchKernelGGL(k_set_words, dim3(1), dim3(2 * DEC_WORDS), 0, d->stream, w, d->words, d->slots[0],
                       d->slots[1], d->d.pos, d->B);
    NC_LAUNCH_CHECK();
    if (lo >= 0) { /* the masked slots' allowed-token rows, lowest to highest */
        const size_t row = (size_t)(d->vocab + 31) / 32 * 4;
        NC_HIP_CHECK(hipMemcpyAsync((uint8_t *)d->allow + lo * row, (uint8_t *)d->host_allow + lo * row,
                                    (hi + 1 - lo) * row, hipMemcpyHostToDevice, d->stream));
    }
}

extern "C" void dec_launch_body(void *handle) {
    Decoder *d = (Decoder *)handle;
    NC_HIP_CHECK(hipGraphLaunch(d->body[d->narrow], d->stream));
}

extern "C" void dec_launch_head(void *handle) {
    Decoder *d = (Decoder *)handle;
    NC_HIP_CHECK(hipGraphLaunch(d->head[d->narrow], d->stream));
}

/* Waits for the launched step: out[b] the token slot b took, out[B + b] its alternative (stale for idle slots). */
extern "C" void dec_tokens(void *handle, int32_t *out) {
    Decoder *d = (Decoder *)handle;
    NC_HIP_CHECK(hipMemcpyAsync(d->host_tokens, d->d.tok, (size_t)d->B * sizeof(int32_t), hipMemcpyDeviceToHost,
                                d->stream));
    NC_HIP_CHECK(hipMemcpyAsync(d->host_tokens + d->B, d->alt, (size_t)d->B * sizeof(int32_t),
                                hipMemcpyDeviceToHost, d->stream));
    NC_HIP_CHECK(hipStreamSynchronize(d->stream));
    memcpy(out, d->host_tokens, 2 * (size_t)d->B * sizeof(int32_t));
}

extern "C" void dec_take_alt(void *handle, int b) {
    Decoder *d = (Decoder *)handle;
    if (b < 0 || b >= d->B) {
        fprintf(stderr, "dec_take_alt: slot %d outside [0, %d)\n", b, d->B);
        abort();
    }
    hipLaunchKernelGGL(k_take_alt, dim3(1), dim3(1), 0, d->stream, d->d.tok, d->alt, b);
    NC_LAUNCH_CHECK();
}
