/* ccdecode.h — C ABI of the MI355X batched ragged decode pass.
 *
 * The library replaces the GPU side of the reference's Runner
 * (web/model/stage.js): one context owns a contiguous range of positions
 * (0 = embedding, 1..L = blocks, L+1 = final norm + LM head), its q8 weights,
 * an int8 paged KV pool, session frames (slots) with page tables, and all
 * scratch. cc_step runs one packed pass over prepared jobs — the reference's
 * Runner.#pass (web/model/stage.js:1314-1481) — and returns per-row top-M
 * candidates or the f16 rows handed downstream.
 *
 * Host policy (queueing, batching rules, admission, eviction, cuts, boundary
 * logs) stays with the caller, as it does in the reference's Runner; the
 * caller is the JS shim (chattorrent_amd/node/runner.js) over the N-API addon,
 * or Python over ctypes. Every entry point returns a cc_status; on failure
 * cc_last_error() holds the message. A context is not reentrant: calls on one
 * context must not overlap (the reference runs jobs one at a time,
 * web/model/stage.js:5, :646-654).
 *
 * Plain C types only. Host buffers are owned by the caller for the duration of
 * the call; the library copies through its own pinned staging.
 */
#ifndef CCDECODE_H
#define CCDECODE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error classes of the reference's Runner, kept per job
 * (web/model/stage.js:930-941 busy, :948-958 / :1073-1079 cold,
 * :1067-1072 stale, :339-345 nospec, :1225-1259 bad job, :1114-1117 pool too
 * small; device loss: web/engine.js:703-744). */
typedef enum cc_status {
    CC_OK = 0,
    CC_BUSY = 1,      /* capacity refusal (no frame / page free now) */
    CC_COLD = 2,      /* the session's cache is not here (evicted or behind) */
    CC_STALE = 3,     /* a duplicate job behind the cache */
    CC_NOSPEC = 4,    /* no speculative replay state (hybrid models only) */
    CC_EARG = 5,      /* a malformed job or call */
    CC_EPOOL = 6,     /* the KV pool cannot hold this context at all */
    CC_EOOM = 7,      /* device allocation failed */
    CC_EDEVICE = 8    /* a HIP error; the context should be destroyed */
} cc_status;

/* Model dimensions: loader.js dimsFromManifest (web/model/loader.js:146-201),
 * checked like model.js checkDims (web/model/model.js:22-40). */
typedef struct cc_dims {
    int32_t hidden, n_layer, n_heads, n_kv_heads, head_dim, ffn, vocab;
    int32_t q8_group;       /* weights: one scale per this many values along K (32) */
    float rms_eps;
    double rope_theta;
    int32_t rope_scaling;   /* 0 none, 1 llama3 (kernels.js:1998-2014) */
    double rs_factor, rs_low_freq, rs_high_freq, rs_orig_max_pos;
    int32_t tied;           /* LM head reads the embedding table */
    /* Hybrid (Qwen3.5-architecture) checkpoints — dimsFromManifest,
     * web/model/loader.js:146-201. rot_dim: RoPE width (partial rotary,
     * kernels.js:1080-1129); 0 means head_dim. hybrid != 0: full_attention
     * blocks also carry attn_gate, q_norm and k_norm (loader.js:543-565), and
     * n_heads*head_dim may differ from hidden. layer_kinds: n_layer entries,
     * CC_FULL_ATTENTION or CC_LINEAR_ATTENTION (NULL: every block full; the
     * array is copied by cc_create). lin_*: Gated DeltaNet's key heads, value
     * heads, key and value head widths, conv width (linear_num_key_heads ..
     * linear_conv_kernel_dim). */
    int32_t rot_dim;
    int32_t hybrid;
    const uint8_t* layer_kinds;
    int32_t lin_nk, lin_nv, lin_dk, lin_dv, lin_conv;
    /* The MTP draft head (model.js:529-576, loader.js:628-638): the
     * vocabulary rows it drafts over (manifest mtp.draft_vocab); 0: none. A
     * context holding the head holds it. */
    int32_t mtp_vocab;
} cc_dims;
enum { CC_FULL_ATTENTION = 0, CC_LINEAR_ATTENTION = 1 };

/* Runner options (web/model/stage.js:107-110). lo/hi: the position range
 * held; n_max: context window; t_max: the most rows one pass carries; slots:
 * full contexts the KV pool holds (pages = slots * ceil(n_max/page));
 * sessions: frames (page tables). */
typedef struct cc_opts {
    int32_t lo, hi;
    int32_t n_max;
    int32_t t_max;
    int32_t slots;
    int32_t sessions;
    int32_t page_tokens;    /* 64 (web/split.js:75) */
    int32_t max_jobs;       /* the most jobs one pass packs */
    int32_t device;
} cc_opts;

typedef struct cc_ctx cc_ctx;

/* Tensor ids for cc_upload / cc_fill_random (HF names). layer = -1 for the
 * model-level tensors. */
enum {
    CC_T_Q = 0, CC_T_K = 1, CC_T_V = 2, CC_T_O = 3, CC_T_GATE = 4, CC_T_UP = 5, CC_T_DOWN = 6,
    CC_T_LN1 = 7, CC_T_LN2 = 8, CC_T_WTE = 9, CC_T_NORM = 10, CC_T_LM_HEAD = 11,
    /* a hybrid checkpoint's full_attention extras (loader.js:543-565):
     * attn_gate q8 [n_heads*head_dim, hidden]; q_norm, k_norm f32 [head_dim] */
    CC_T_ATTN_GATE = 12, CC_T_Q_NORM = 13, CC_T_K_NORM = 14,
    /* linear_attention blocks (loader.js:567-590, tools/convert_hf.py:188-219):
     * in_proj_q/k q8 [keyDim, hidden], in_proj_v/z q8 [valueDim, hidden],
     * in_proj_b/a q8 [nV, hidden], conv1d_q/k f32 [keyDim, conv],
     * conv1d_v f32 [valueDim, conv], gate_params f32 [2*nV] (A_log, then
     * dt_bias), gated_norm f32 [Dv], out_proj q8 [hidden, valueDim] */
    CC_T_IN_Q = 15, CC_T_IN_K = 16, CC_T_IN_V = 17, CC_T_IN_Z = 18, CC_T_IN_B = 19, CC_T_IN_A = 20,
    CC_T_CONV_Q = 21, CC_T_CONV_K = 22, CC_T_CONV_V = 23, CC_T_GATE_PARAMS = 24, CC_T_GATED_NORM = 25,
    CC_T_OUT_PROJ = 26,
    /* the MTP head (loader.js:633-634): enorm, hnorm, mtp_norm f32 [hidden];
     * fc_e, fc_h q8 [hidden, hidden]; embed_draft, head_draft q8
     * [mtp_vocab, hidden]. Its full-attention block's tensors are the block
     * ids above at layer CC_LAYER_MTP. */
    CC_T_MTP_ENORM = 27, CC_T_MTP_HNORM = 28, CC_T_MTP_FC_E = 29, CC_T_MTP_FC_H = 30, CC_T_MTP_NORM = 31,
    CC_T_MTP_EMBED = 32, CC_T_MTP_HEAD = 33
};
enum { CC_LAYER_MTP = -2 };
enum { CC_SCALES_F16 = 0, CC_SCALES_F32 = 1 };

/* new Runner(device, d, w, {...}) — web/model/stage.js:107-238. */
cc_status cc_create(const cc_dims* dims, const cc_opts* opts, cc_ctx** out);
void cc_destroy(cc_ctx* ctx);
const char* cc_last_error(const cc_ctx* ctx);

/* uploadQ8(device, int8Bytes, scales, group) — web/model/kernels.js:122-126;
 * norms (tensor LN1/LN2/NORM) are f32 `data` with n = hidden and no scales,
 * and so are the hybrid f32 tensors (Q_NORM .. GATED_NORM, n = their size).
 * q8 tensors: `data` int8 [N, K] row-major, `scales` [N, ceil(K/group)] as
 * f16 bits or f32 (rounded to the device's f16 scale). `group` is any
 * multiple of 32 (the reference's converter writes 64,
 * tools/convert_hf.py:493): a scale covering group/32 of the device's
 * 32-wide groups is given to each of them, which is exact. */
cc_status cc_upload(cc_ctx* ctx, int32_t layer, int32_t tensor, const void* data, size_t n,
                    const void* scales, size_t ns, int32_t scale_dtype, int32_t group);

/* Synthetic weights on the device from the counter-based generator shared
 * with the test oracle (no reference counterpart: the reference's random
 * models are randomWeights, web/model/model.js:697-717). On a hybrid model
 * (and for the MTP head) this is for timing only: the Gated DeltaNet's f32
 * parameters take fixed values (conv taps 0.25, A_log -1, dt_bias 0) that
 * the oracle does not mirror; parity tests upload their weights. */
cc_status cc_fill_random(cc_ctx* ctx, uint64_t seed);

/* One prepared job of a pass (the fields #prepare hands #pass,
 * web/model/stage.js:1195-1308). `ids` when the pass enters at position 0,
 * else `hidden` (n*hidden f16 bits). `sampled`: rows the head samples — 1
 * (the last row) or n (a verify); 0 when the pass does not reach the head. */
typedef struct cc_job {
    int32_t slot;
    int32_t past;
    int32_t n;
    int32_t sampled;
    const int32_t* ids;
    const uint16_t* hidden;
    /* Speculative decoding through linear_attention blocks (stage.js:1248-1283,
     * model.js:447-470 restoreSpec / snapSpec). snap != 0: a verify job
     * (n <= 8 rows); its blocks keep the state it starts from and its rows'
     * projections. rollback != 0: the session's last job here was a verify
     * from `base`; this job continues at past = base + keep (0 <= keep <= that
     * verify's n): the blocks go back to the verify's starting state and
     * re-run its first `keep` rows before this job's own. Zero-initialised
     * fields mean neither. */
    int32_t snap;
    int32_t rollback;
    int32_t keep;
    /* The job's session drafts with the MTP head (stage.js:1287-1293): at a
     * context holding it, the MTP layer's KV rows past..past+n-1 are filled
     * from the job's `ids` (given whatever the entry position) paired with
     * the trunk's hidden rows one position earlier; a job that samples
     * nothing keeps its last row for the next job (stage.js:1408-1421). */
    int32_t mtp;
} cc_job;

/* Runner.#pass — web/model/stage.js:1314-1481. Runs positions [at, to) for
 * `njobs` jobs packed in order. Pages for rows past..past+n-1 are taken from
 * the pool on the device in job order (model.js ensurePages replayed).
 * Outputs: when `to` is past the last block (the head), `top_vals`/`top_ids`
 * receive `topk` candidates per sampled row (sampled rows in job order, best
 * first, ties to the lower id); otherwise `hidden_out` receives every row as
 * f16 bits [T, hidden]. `status` (optional, njobs) is set per job. */
cc_status cc_step(cc_ctx* ctx, const cc_job* jobs, int32_t njobs, int32_t at, int32_t to,
                  int32_t topk, float* top_vals, uint32_t* top_ids, uint16_t* hidden_out,
                  int32_t* status);

/* `steps` greedy passes of Runner.#pass (web/model/stage.js:1314-1481) run
 * back to back on the device, the route's closed decode loop
 * (web/route.js:865-952) without a host round trip between passes: every
 * job is one row, sampled; pass k runs each job at past + k with the token
 * pass k-1 sampled (column 0 of its candidates; pass 0 takes jobs[j].ids[0]),
 * and packs its rows and attention work on the device. Each pass takes the
 * pages its jobs newly need, job by job, as a cc_step of that pass would, so
 * the frames' page tables and the pool end as after `steps` cc_step calls
 * (CC_BUSY, before anything runs, when the pool cannot supply them).
 * Outputs: top_vals / top_ids [steps][njobs][topk], best first. Each pass's
 * results equal cc_step's for the same jobs. A context holding every position of a full-attention model
 * without an MTP head. */
cc_status cc_decode_steps(cc_ctx* ctx, const cc_job* jobs, int32_t njobs, int32_t steps, int32_t topk,
                          float* top_vals, uint32_t* top_ids);

/* After sampling `token` from row `row` of the last pass (Runner.#mtpAfter,
 * web/model/stage.js:296-320): the session keeps that row's hidden state
 * (row -1: keep the one it has) and, for k_drafts > 0 (at most 7), the MTP
 * head chains that many drafts after `token` at positions pos..
 * (model.js:567-576 mtpChain: each step's argmax over the draft vocabulary,
 * lowest id on a tie, is the next step's token). The MTP layer's KV rows
 * written there are speculative; the next job's fill rewrites them. Pages
 * are taken for pos + k_drafts tokens. `drafts` receives k_drafts ids. */
cc_status cc_mtp_draft(cc_ctx* ctx, int32_t slot, int32_t row, int32_t token, int32_t pos, int32_t k_drafts,
                       uint32_t* drafts);

/* Runner.#release / freePages — web/model/stage.js:842-874,
 * web/model/model.js:204-211: the slot's pages return to the pool. */
cc_status cc_release(cc_ctx* ctx, int32_t slot);

/* Frame pages the slot holds (the frame's `owned` length). */
int32_t cc_slot_pages(const cc_ctx* ctx, int32_t slot);
int32_t cc_free_pages(const cc_ctx* ctx);

/* Fill rows 0..tokens-1 of a slot with random int8 KV (codes uniform in
 * ±127, one f16 scale ~U(0.005, 0.02) per token and kv head), taking pages
 * as a job would. `key` names the chat in the generator index. */
cc_status cc_fill_random_kv(cc_ctx* ctx, int32_t slot, int32_t tokens, uint64_t seed, uint64_t key);

/* Debug readback in the reference's row layout (web/model/kernels.js:999-1022:
 * D/4 code words then D/QB f32 scales per row): rows t0..t1-1 of one kv head,
 * which = 0 for K, 1 for V, `layer` a held block index. */
cc_status cc_read_kv(cc_ctx* ctx, int32_t layer, int32_t which, int32_t slot, int32_t head,
                     int32_t t0, int32_t t1, uint32_t* out);
cc_status cc_write_kv(cc_ctx* ctx, int32_t layer, int32_t which, int32_t slot, int32_t head,
                      int32_t t0, int32_t t1, const uint32_t* rows);
cc_status cc_read_pages(cc_ctx* ctx, int32_t slot, uint32_t* out, int32_t n);

/* The last pass's full logits rows [rows, vocab] f32 (the sampled rows of a
 * pass that reached the head), for parity checks: the reference reads back
 * whole rows when a sampler needs them (web/model/stage.js:1428-1436). */
cc_status cc_read_logits(cc_ctx* ctx, int32_t rows, float* out);

/* Stats (Runner.counts / vramBytes, web/model/stage.js:219-259). */
typedef struct cc_stats {
    uint64_t vram_bytes;
    uint64_t weight_bytes;
    uint64_t kv_bytes;
    uint64_t scratch_bytes;
    int64_t passes;
    int64_t rows;
    double last_pass_ms;
} cc_stats;
cc_status cc_stats_get(const cc_ctx* ctx, cc_stats* out);

/* Per-kernel timing with HIP events on the context's stream (the
 * reference's gpuprof.js level 2, web/model/gpuprof.js:1-12, re-done for
 * HIP). While enabled, each cc_step, after its own work, launches each class
 * below again for every block of the step, back-to-back between one event
 * pair (so no marker sits between launches); cc_profile_read returns the
 * summed milliseconds, the launch count and the algorithmic HBM bytes of
 * those launches (q8 weights at 1.0625 B per weight; KV rows at
 * D + 4*D/32 B). The step's results are unchanged. Enabling resets the sums. */
enum { CC_K_QKV = 0, CC_K_O = 1, CC_K_GU = 2, CC_K_DOWN = 3, CC_K_HEAD = 4, CC_K_ATTN = 5, CC_K_COUNT = 6 };
cc_status cc_profile(cc_ctx* ctx, int32_t enable);
cc_status cc_profile_read(const cc_ctx* ctx, int32_t kind, double* ms, int64_t* launches, double* bytes);

/* ---- Kernel-level entry points (one reference kernel each), used by the
 * parity tests to hold each GPU kernel to the oracle on identical inputs. All
 * pointers are host memory. ---- */

/* matmulNobias for q8 — web/model/kernels.js:1874-1914. Y[M,N] = X[M,K] W^T. */
cc_status cc_op_matmul_q8(cc_ctx* ctx, const float* X, int32_t M, int32_t K,
                          const int8_t* W, const uint16_t* scales_f16, int32_t N, float* Y);
/* store_kv — web/model/kernels.js:1960-1973, into `slot`'s pages of block
 * `layer`: src [T_new, nKV*D] f32; rope != 0 rotates (K), else V. */
cc_status cc_op_store_kv(cc_ctx* ctx, int32_t layer, int32_t which, int32_t slot,
                         const float* src, int32_t T_new, int32_t T_past);
/* round_f16 — web/model/kernels.js:2100-2105. In place on n floats. */
cc_status cc_op_round_f16(cc_ctx* ctx, float* a, int64_t n);
/* topkRows — web/model/kernels.js:2129-2144: rows x V logits → M pairs. */
cc_status cc_op_topk(cc_ctx* ctx, const float* logits, int32_t rows, int32_t V, int32_t M,
                     float* vals, uint32_t* ids);
/* No counterpart in the reference: an allocation-free cc_op_topk for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). `logits` [rows, V] f32,
 * `vals` and `ids` [rows, M] are DEVICE pointers the caller owns; the stages'
 * keys go to a static 4 MiB scratch array per GPU (TOPK_SCRATCH_KEYS keys),
 * and calls needing more are refused with CC_EARG. The first stage keeps
 * rows * ceil(V/4096) * M keys and the next one far fewer: at M = 1 and
 * V = 2^20 a call needs rows * 257 keys, so up to 2040 rows fit; at M = 256
 * and V = 262144, 30 rows.
 * Runs asynchronously on
 * `stream` (a hipStream_t; NULL: the context's stream): the caller
 * synchronises before reading `vals`/`ids`. Calls no hipMalloc, hipFree or
 * allocating routine. Every call on one GPU shares that GPU's scratch, so
 * calls that overlap on one GPU (different streams or contexts) race. */
cc_status cc_topk_noalloc(cc_ctx* ctx, const float* logits, int32_t rows, int32_t V, int32_t M, float* vals,
                          uint32_t* ids, void* stream);
/* rmsnorm — web/model/kernels.js:1927-1932. */
cc_status cc_op_rmsnorm(cc_ctx* ctx, const float* x, const float* w, int32_t T, int32_t H,
                        float* y);
/* attend (web/model/model.js:321-351) for one job of block `layer` whose K/V
 * rows are already stored: q [n, nH*D] f32 (before RoPE) -> out [n, nH*D]. */
cc_status cc_op_attend(cc_ctx* ctx, int32_t layer, int32_t slot, const float* q, int32_t n,
                       int32_t past, float* out);

#ifdef __cplusplus
}
#endif
#endif
