// C ABI of the MI355X batched ragged decode pass (include/ccdecode.h).
//
// A context plays the GPU half of the reference's Runner
// (web/model/stage.js): it owns the held positions' weights, the paged int8
// KV pool with its page tables and free stack, and the scratch of one pass.
// cc_step is Runner.#pass (web/model/stage.js:1314-1481): it packs the jobs'
// rows, takes their pages, runs the embedding, the blocks and the head, and
// returns candidates or rows. The caller keeps the Runner's policy (queue,
// batching, admission, eviction); the library validates every job before any
// device work and reports a status per job.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ccdecode.h"
#include "common.h"
#include "kernels.h"

namespace {

constexpr int TOPK_MAX = 256;   // web/model/sampling.js:125

struct Layer {
    int kind = CC_FULL_ATTENTION;
    QTensor qkv, o, gu, down;
    float* ln1 = nullptr;
    float* ln2 = nullptr;
    uint8_t* kpool = nullptr;
    uint8_t* vpool = nullptr;
    // a hybrid checkpoint's full_attention extras (attn_gate rides in qkv)
    float* qn = nullptr;
    float* kn = nullptr;
    // linear_attention: fused in_proj (q|k|v|z|b|a), out_proj, conv weights
    // [convDim][4], gate_params [2*nV], gated_norm [Dv], per-session state
    QTensor lin, out;
    float* conv = nullptr;
    float* gp = nullptr;
    float* gnorm = nullptr;
    float* state = nullptr;
};

int ceil_div(int a, int b) { return (a + b - 1) / b; }

constexpr int MTP_STEPS_MAX = 7;   // SPEC_COLS - 1 drafts (stage.js:303-304)
constexpr int PPW_NARROW = 2;   // pages per attention item for narrow K/V rows (nKV * D <= 512)

}  // namespace

struct cc_ctx {
    cc_dims d{};
    cc_opts o{};
    int group = 0, D = 0, rot = 0, L0 = 0, L1 = 0;
    bool embed = false, head = false;
    // hybrid checkpoints: block kinds (model numbering), Gated DeltaNet shape,
    // q width n_heads*head_dim, and the linear blocks' scratch
    bool hybrid = false;
    std::vector<uint8_t> kinds;
    LinGeom lg{};
    int qdim = 0;
    float* lraw = nullptr;         // [t_max][lg.W] conv outputs, z, b, a
    float* lcore = nullptr;        // [t_max][valueDim] recurrence output
    uint4* xp_v = nullptr;         // operand for K = valueDim
    float* gbuf = nullptr;         // [t_max][qdim] output-gate values
    float* lrep = nullptr;         // [max_jobs][LIN_SPEC_ROWS][lg.lrep_w] rows a rollback re-runs
    float* lring = nullptr;        // [max_jobs][K-1][convDim] the ring each job starts from (long jobs)
    bool any_linear = false;
    // per session: its last job here was a verify from spec_base of spec_n rows
    std::vector<int> spec_base, spec_n;
    std::vector<int> fed;          // per session: rows its recurrent blocks hold
    // the MTP draft head (model.js:529-576), held with the LM head
    bool mtp = false;
    Layer mtpL;                    // its full-attention block, own KV pools
    QTensor fc_e, fc_h, embed_draft, head_draft;
    float* enorm = nullptr;
    float* hnorm = nullptr;
    float* mtp_norm = nullptr;
    float* mtpH = nullptr;         // [sessions][H] the trunk row a session's next MTP row pairs with
    float* mx = nullptr;           // [t_max][H] the MTP block's rows
    float* mtp_in = nullptr;       // [t_max][H] the hidden rows paired with the tokens
    float* mtp_e = nullptr;        // [t_max][H] draft embeddings
    uint4* xp_e = nullptr;         // operands of enorm(e) and hnorm(h)
    uint4* xp_hh = nullptr;
    float* mtp_logits = nullptr;   // head_draft planes for one row
    uint8_t* d_chain = nullptr;    // draft chain metadata (device) and its pinned staging
    uint8_t* h_chain = nullptr;
    size_t chain_step = 0;         // bytes per chain step
    int last_T = 0;                // rows the last pass left in x
    std::vector<Layer> layers;
    QTensor wte, lm_head;
    float* norm = nullptr;
    float* tbl = nullptr;
    int tbl_cap = 0;
    KVGeom geom{};
    int n_pages = 0, max_pages = 0;
    uint32_t* page_table = nullptr;
    uint32_t* free_stack = nullptr;
    std::vector<int> owned;
    int top = 0;
    // scratch
    int mt_alloc = 0;              // operand m-tiles allocated (even)
    float* x = nullptr;            // residual [t_max][H]
    uint4* xp_h = nullptr;         // operand for K = hidden
    uint4* xp_o = nullptr;         // operand for K = nH*D
    uint4* xp_f = nullptr;         // operand for K = ffn
    float* ssp = nullptr;          // rmsnorm partial sums of squares [rows][RW_SMAX]
    float* part = nullptr;
    size_t part_floats = 0;
    int ncu = 0;                   // compute units: the matmul's workgroup count
    uint4* qp = nullptr;
    size_t qp_units = 0;
    float* apart = nullptr;
    size_t apart_floats = 0;
    int ppw = 8;                   // pages per attention work item
    AttnSched attn;                // attention launches' block counters
    AttnItem* d_items = nullptr;
    size_t items_cap = 0;
    float* logits = nullptr;       // LM-head planes [P][rows][vocab]
    int head_planes = 1, head_rows = 0;
    uint64_t* tk_a = nullptr;
    uint64_t* tk_scratch = nullptr;   // this device's static scratch (cc_topk_noalloc)
    uint64_t* tk_b = nullptr;
    float* d_vals = nullptr;
    uint32_t* d_ids = nullptr;
    // cc_decode_steps' per-step outputs, grown to the largest call
    float* dec_vals = nullptr;
    uint32_t* dec_ids = nullptr;
    size_t dec_cap = 0;
    int32_t* dec_plan = nullptr;   // cc_decode_steps: every pass's page pops
    size_t dec_plan_cap = 0;       // (int32 entries)
    uint16_t* d_hbits = nullptr;
    // per-step metadata (device) and its pinned host staging
    uint8_t* d_meta = nullptr;
    uint8_t* h_meta = nullptr;
    size_t meta_bytes = 0;
    void* h_out = nullptr;
    size_t out_bytes = 0;
    hipStream_t stream = nullptr;
    std::string err;
    uint64_t weight_bytes = 0, kv_bytes = 0, scratch_bytes = 0;
    int64_t passes = 0, rows = 0;
    double last_ms = 0;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::vector<void*> allocs;
    // opt-in per-kernel profile (cc_profile)
    bool prof = false;
    std::vector<hipEvent_t> pev;               // event pool, pairs
    struct Mark { int kind; int e0, e1; int n; double bytes; };
    std::vector<Mark> marks;
    double prof_ms[CC_K_COUNT] = {0};
    int64_t prof_n[CC_K_COUNT] = {0};
    double prof_bytes[CC_K_COUNT] = {0};
};

namespace {

cc_status fail(cc_ctx* c, cc_status s, const std::string& msg) {
    if (c) c->err = msg;
    return s;
}

#define HIPCHK(expr)                                                                               \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess)                                                                      \
            return fail(ctx, e_ == hipErrorOutOfMemory ? CC_EOOM : CC_EDEVICE,                     \
                        std::string(#expr) + ": " + hipGetErrorString(e_));                        \
    } while (0)

// Device allocations are zeroed on the context's own stream: it is a
// non-blocking stream, so work on the null stream would not be ordered
// against the fills and copies that follow.
template <class T>
hipError_t dalloc(cc_ctx* ctx, T** p, size_t bytes, uint64_t* acct) {
    void* v = nullptr;
    hipError_t e = hipMalloc(&v, bytes ? bytes : 16);
    if (e != hipSuccess) return e;
    e = hipMemsetAsync(v, 0, bytes ? bytes : 16, ctx->stream);
    if (e != hipSuccess) return e;
    ctx->allocs.push_back(v);
    if (acct) *acct += bytes;
    *p = (T*)v;
    return hipSuccess;
}

// Frees a buffer dalloc made (nullptr: nothing) once the context's stream
// has finished with it, and drops it from the context's list and account.
template <class T>
hipError_t dfree(cc_ctx* ctx, T* p, size_t bytes, uint64_t* acct) {
    if (!p) return hipSuccess;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return e;
    for (size_t i = 0; i < ctx->allocs.size(); i++)
        if (ctx->allocs[i] == (void*)p) {
            ctx->allocs[i] = ctx->allocs.back();
            ctx->allocs.pop_back();
            if (acct) *acct -= bytes;
            return hipFree((void*)p);
        }
    return hipSuccess;
}

hipError_t alloc_q(cc_ctx* ctx, QTensor& q, int N, int K) {
    q.N = N;
    q.K = K;
    q.Nt = ceil_div(ceil_div(N, 16), 2) * 2;   // tile pairs
    q.KU = ceil_div(K, 64);
    q.P = lx_planes_for(N, K, ctx->ncu);
    return dalloc(ctx, &q.codes, (size_t)q.Nt * q.KU * (LX_REC / 2), &ctx->weight_bytes);
}

void build_rope_table(cc_ctx* ctx, std::vector<float>& t) {
    // web/model/kernels.js:2016-2045 ropeTable: f64 cos/sin, rounded to f32.
    const int half = ctx->rot / 2;
    t.assign((size_t)ctx->tbl_cap * ctx->rot, 0.0f);
    const cc_dims& d = ctx->d;
    for (int i = 0; i < half; i++) {
        double inv = std::pow(d.rope_theta, -(2.0 * i) / (double)ctx->rot);
        if (d.rope_scaling == 1) {
            const double PI = 3.14159265358979323846;
            double wavelen = (2.0 * PI) / inv;
            double lowW = d.rs_orig_max_pos / d.rs_low_freq, highW = d.rs_orig_max_pos / d.rs_high_freq;
            if (wavelen < highW) {
            } else if (wavelen > lowW) {
                inv = inv / d.rs_factor;
            } else {
                double smooth = (d.rs_orig_max_pos / wavelen - d.rs_low_freq) / (d.rs_high_freq - d.rs_low_freq);
                inv = smooth * inv + (1.0 - smooth) * (inv / d.rs_factor);
            }
        }
        for (int pos = 0; pos < ctx->tbl_cap; pos++) {
            double ang = (double)pos * inv;
            t[((size_t)pos * half + i) * 2] = (float)std::cos(ang);
            t[((size_t)pos * half + i) * 2 + 1] = (float)std::sin(ang);
        }
    }
}

cc_status check_dims(cc_ctx* ctx, const cc_dims& d, const cc_opts& o) {
    // web/model/model.js:22-40 checkDims, plus what these kernels assume.
    if (d.hidden <= 0 || d.n_layer <= 0 || d.n_heads <= 0 || d.n_kv_heads <= 0 || d.head_dim <= 0 ||
        d.ffn <= 0 || d.vocab <= 0)
        return fail(ctx, CC_EARG, "every dimension must be positive");
    const bool hyb = d.hybrid != 0;
    if (!hyb && d.n_heads * d.head_dim != d.hidden)
        return fail(ctx, CC_EARG, "n_heads*head_dim (" + std::to_string(d.n_heads * d.head_dim) +
                                      ") != hidden (" + std::to_string(d.hidden) + ")");
    const int rot = d.rot_dim ? d.rot_dim : d.head_dim;
    if (rot < 2 || rot > d.head_dim || rot % 2)
        return fail(ctx, CC_EARG, "rot_dim must be even and at most head_dim (RoPE's split-half pairing)");
    bool any_linear = false;
    if (d.layer_kinds) {
        for (int i = 0; i < d.n_layer; i++) {
            if (d.layer_kinds[i] > CC_LINEAR_ATTENTION)
                return fail(ctx, CC_EARG, "layer_kinds holds a kind other than full or linear attention");
            any_linear = any_linear || d.layer_kinds[i] == CC_LINEAR_ATTENTION;
        }
    }
    if (any_linear && !hyb) return fail(ctx, CC_EARG, "linear_attention blocks need a hybrid checkpoint");
    if (d.mtp_vocab < 0 || d.mtp_vocab > d.vocab) return fail(ctx, CC_EARG, "mtp_vocab must be 0..vocab");
    if (any_linear) {
        // loader.js:225-230, plus the Gated DeltaNet kernels' shapes
        if (d.lin_nk <= 0 || d.lin_nv <= 0 || d.lin_nv % d.lin_nk)
            return fail(ctx, CC_EARG, "linear_num_value_heads (" + std::to_string(d.lin_nv) +
                                          ") not divisible by linear_num_key_heads (" + std::to_string(d.lin_nk) + ")");
        if (d.lin_dk != 16 && d.lin_dk != 32 && d.lin_dk != 64 && d.lin_dk != 128)
            return fail(ctx, CC_EARG, "linear_key_head_dim must be 16, 32, 64 or 128");
        if (d.lin_dv <= 0 || d.lin_dv % 16 || d.lin_dv > 512)
            return fail(ctx, CC_EARG, "linear_value_head_dim must be a multiple of 16, at most 512");
        if (d.lin_conv != LIN_CONV_K) return fail(ctx, CC_EARG, "linear_conv_kernel_dim must be 4");
    }
    if (d.n_heads % d.n_kv_heads != 0) return fail(ctx, CC_EARG, "n_heads not divisible by n_kv_heads");
    if (d.head_dim != 64 && d.head_dim != 128 && d.head_dim != 256)
        return fail(ctx, CC_EARG, "head_dim must be 64, 128 or 256 (the int8 KV blocks are 32 wide)");
    if (d.q8_group != 32) return fail(ctx, CC_EARG, "q8 weights must use one scale per 32 values");
    // Fused q|k|v and gate|up start each part on a tile pair (32 rows).
    if (d.hidden % 64 || d.ffn % 32) return fail(ctx, CC_EARG, "hidden must be a multiple of 64, ffn of 32");
    if ((d.n_kv_heads * d.head_dim) % 32) return fail(ctx, CC_EARG, "n_kv_heads*head_dim must be a multiple of 32");
    if (d.hidden > RESID_NORM_HMAX)
        return fail(ctx, CC_EARG, "hidden above " + std::to_string(RESID_NORM_HMAX) + " is not supported");
    // The matmul addresses a weight with 32-bit byte offsets.
    const double H = d.hidden, F = d.ffn;
    const double qd = (double)d.n_heads * d.head_dim;
    const double big = std::max({(double)d.vocab * H, 2.0 * F * H, F * H,
                                 (2.0 * qd + 2.0 * d.n_kv_heads * d.head_dim) * H,
                                 (2.0 * d.lin_nk * d.lin_dk + 2.0 * d.lin_nv * d.lin_dv + 2.0 * d.lin_nv + 32) * H}) *
                       1.0625;
    if (big > 2.0e9) return fail(ctx, CC_EARG, "a weight above 2 GB is not supported");
    if ((double)o.t_max * std::max(d.vocab, 2 * d.ffn) * 4.0 > 2.0e9)
        return fail(ctx, CC_EARG, "t_max rows of logits must stay under 2 GB");
    const int positions = d.n_layer + 2;
    if (o.lo < 0 || o.hi > positions || o.lo >= o.hi) return fail(ctx, CC_EARG, "bad position range");
    if (o.n_max <= 0 || o.t_max <= 0 || o.slots <= 0 || o.sessions <= 0 || o.max_jobs <= 0)
        return fail(ctx, CC_EARG, "n_max, t_max, slots, sessions and max_jobs must be positive");
    if (o.max_jobs > PACK_MAX_JOBS)
        return fail(ctx, CC_EARG, "max_jobs is at most " + std::to_string(PACK_MAX_JOBS));
    if (o.page_tokens != 64) return fail(ctx, CC_EARG, "page_tokens must be 64 (web/split.js:75)");
    if (o.t_max > 4096) return fail(ctx, CC_EARG, "t_max above 4096 rows is not supported");
    // attention chunks of ceil(pages/512) pages, at most 64 (one page index a lane)
    if ((int64_t)o.n_max > (int64_t)64 * 512 * 64) return fail(ctx, CC_EARG, "n_max above 2097152 tokens is not supported");
    return CC_OK;
}

struct StepPlan {
    // nitems: attention partials (job, kv head, m-tile, chunk); nlaunch: the
    // item list k_attn takes (blocks of m-tiles padded to 4)
    int T = 0, S = 0, nitems = 0, ncwg = 0, nlaunch = 0;
    int multi = 0;   // a job of several Q m-tiles (attention's shared-page blocks)
    std::vector<JobDev> jobs;
    std::vector<AttnItem> items;
    std::vector<int32_t> row_job, plan, head_rows, cwg;
    size_t qp_units = 0, apart_floats = 0;
    double kv_bytes = 0;   // K and V rows one layer's attention reads (reference row size)
};

// Per-step metadata. First what the host writes each pass (the page plan,
// the jobs for the device packer, ids | hidden rows, the MTP fill's rows),
// copied in one transfer; then what the device packer builds (jobs, items,
// row_job, head_rows, combine workgroups (job, kv head, m-tile)).
struct MetaLayout {
    size_t plan, pack, ids, mtp_jobs, mtp_row_job, mtp_src, mtp_ids, hidden;
    size_t jobs, items, row_job, head_rows, cwg, total;
};

// (job, kv head, m-tile) triples a pass can hold.
size_t max_cwg_for(const cc_ctx* ctx) {
    return (size_t)ctx->geom.nKV * (ceil_div(ctx->o.t_max * ctx->group, 16) + ctx->o.max_jobs);
}

MetaLayout meta_layout(const cc_ctx* ctx) {
    const int max_jobs = ctx->o.max_jobs, t_max = ctx->o.t_max, H = ctx->d.hidden;
    MetaLayout m{};
    size_t at = 0;
    auto take = [&](size_t bytes) { size_t r = at; at += (bytes + 255) & ~(size_t)255; return r; };
    m.plan = take(16 * (size_t)max_jobs);
    m.pack = take(sizeof(PackJob) * max_jobs);
    m.ids = take(4 * (size_t)t_max);
    // the MTP fill's rows (the MTP jobs' rows, packed): jobs, row -> job,
    // hidden-row source (x row, or -1 - slot for the session's kept row), ids
    m.mtp_jobs = take(sizeof(JobDev) * max_jobs);
    m.mtp_row_job = take(4 * (size_t)t_max);
    m.mtp_src = take(4 * (size_t)t_max);
    m.mtp_ids = take(4 * (size_t)t_max);
    m.hidden = take(2 * (size_t)t_max * H);
    m.jobs = take(sizeof(JobDev) * max_jobs);
    m.items = take(sizeof(AttnItem) * ctx->items_cap);
    m.row_job = take(4 * (size_t)t_max);
    m.head_rows = take(4 * (size_t)t_max);
    m.cwg = take(12 * max_cwg_for(ctx));
    m.total = at;
    return m;
}

// Profile marks: one event pair around n back-to-back launches of one class,
// resolved after the step's synchronisation. The events are for timing only
// (no system-scope fence, whose cache writeback would stall the kernels next
// to them).
template <class F>
void prof_mark(cc_ctx* ctx, int kind, int n, double bytes, F&& launches) {
    const int e = (int)ctx->marks.size() * 2;
    while ((int)ctx->pev.size() < e + 2) {
        hipEvent_t ev;
        if (hipEventCreateWithFlags(&ev, hipEventDisableSystemFence) != hipSuccess) return;
        ctx->pev.push_back(ev);
    }
    // a mark whose events cannot be recorded is left out of the profile
    const bool a = hipEventRecord(ctx->pev[e], ctx->stream) == hipSuccess;
    launches();
    const bool b = hipEventRecord(ctx->pev[e + 1], ctx->stream) == hipSuccess;
    if (a && b) ctx->marks.push_back(cc_ctx::Mark{kind, e, e + 1, n, bytes});
}

void prof_collect(cc_ctx* ctx) {
    for (const auto& m : ctx->marks) {
        float ms = 0;
        if (hipEventElapsedTime(&ms, ctx->pev[m.e0], ctx->pev[m.e1]) == hipSuccess) {
            ctx->prof_ms[m.kind] += ms;
            ctx->prof_n[m.kind] += m.n;
            ctx->prof_bytes[m.kind] += m.bytes;
        }
    }
    ctx->marks.clear();
}

double qbytes(const QTensor& q) { return (double)q.N * q.K * (1.0 + 2.0 / 32.0); }

// Attention work items a pass can hold: every (kv head, m-tile) of every job
// times the most chunks of `ppw` pages a frame has.
size_t max_items_for(const cc_ctx* ctx) {
    // a job of several m-tiles pads each (kv head, chunk) to whole blocks of 4
    const size_t mtiles = (size_t)ctx->geom.nKV * (ceil_div(ctx->o.t_max * ctx->group, 16) + 4 * ctx->o.max_jobs);
    return mtiles * ceil_div(ctx->max_pages, ctx->ppw) + 16;
}

}  // namespace

extern "C" {

const char* cc_last_error(const cc_ctx* ctx) { return ctx ? ctx->err.c_str() : "no context"; }

void cc_destroy(cc_ctx* ctx) {
    if (!ctx) return;
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (void* p : ctx->allocs) (void)hipFree(p);
    if (ctx->h_meta) (void)hipHostFree(ctx->h_meta);
    if (ctx->h_out) (void)hipHostFree(ctx->h_out);
    if (ctx->h_chain) (void)hipHostFree(ctx->h_chain);
    if (ctx->ev0) (void)hipEventDestroy(ctx->ev0);
    if (ctx->ev1) (void)hipEventDestroy(ctx->ev1);
    for (hipEvent_t e : ctx->pev) (void)hipEventDestroy(e);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

cc_status cc_create(const cc_dims* dims, const cc_opts* opts, cc_ctx** out) {
    if (!dims || !opts || !out) return CC_EARG;
    *out = nullptr;
    cc_ctx* ctx = new cc_ctx();
    ctx->d = *dims;
    ctx->o = *opts;
    ctx->d.layer_kinds = nullptr;   // the caller's array is copied below, once checked
    cc_status st = check_dims(ctx, *dims, *opts);
    if (st != CC_OK) {
        *out = ctx;   // the caller reads the message, then destroys
        return st;
    }
    ctx->kinds.assign(dims->n_layer, (uint8_t)CC_FULL_ATTENTION);
    if (dims->layer_kinds) ctx->kinds.assign(dims->layer_kinds, dims->layer_kinds + dims->n_layer);
    ctx->d.layer_kinds = ctx->kinds.data();
    const cc_dims& d = ctx->d;
    const cc_opts& o = ctx->o;
    {
        hipError_t e = hipSetDevice(o.device);
        if (e != hipSuccess) {
            *out = ctx;
            return fail(ctx, CC_EDEVICE, std::string("hipSetDevice: ") + hipGetErrorString(e));
        }
    }
    auto body = [&]() -> cc_status {
        HIPCHK(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
        // the allocation-free top-k's scratch address on this device (looked up once per device)
        HIPCHK(topk_scratch_setup(o.device, &ctx->tk_scratch));
        {
            hipDeviceProp_t prop;
            HIPCHK(hipGetDeviceProperties(&prop, o.device));
            ctx->ncu = std::max(1, prop.multiProcessorCount);
        }
        HIPCHK(dalloc(ctx, &ctx->attn.ctr, 2 * sizeof(uint32_t), &ctx->scratch_bytes));
        ctx->attn.ncu = ctx->ncu;
        HIPCHK(hipEventCreate(&ctx->ev0));
        HIPCHK(hipEventCreate(&ctx->ev1));
        ctx->group = d.n_heads / d.n_kv_heads;
        ctx->D = d.head_dim;
        ctx->rot = d.rot_dim ? d.rot_dim : d.head_dim;
        ctx->hybrid = d.hybrid != 0;
        ctx->qdim = d.n_heads * d.head_dim;
        {
            // Gated DeltaNet geometry (loader.js:185-195 d.linear)
            LinGeom& lg = ctx->lg;
            lg.nK = d.lin_nk;
            lg.nV = d.lin_nv;
            lg.Dk = d.lin_dk;
            lg.Dv = d.lin_dv;
            lg.K4 = LIN_CONV_K;
            lg.group = d.lin_nk > 0 ? d.lin_nv / d.lin_nk : 1;
            lg.keyDim = d.lin_nk * d.lin_dk;
            lg.valueDim = d.lin_nv * d.lin_dv;
            lg.convDim = 2 * lg.keyDim + lg.valueDim;
            lg.nVp = 16 * ceil_div(std::max(d.lin_nv, 0), 16);
            lg.W = lg.convDim + lg.valueDim + 2 * lg.nV;
            lg.N = 2 * lg.keyDim + 2 * lg.valueDim + 2 * lg.nVp;
            lg.hist_off = (size_t)lg.nV * lg.Dk * lg.Dv;
            lg.blk = lg.hist_off + (size_t)(LIN_CONV_K - 1) * lg.convDim;
            lg.rep_w = 2 * lg.convDim + 2 * lg.nV;
            lg.lrep_w = lg.convDim + 2 * lg.nV;
            lg.rep_off = 2 * lg.blk;
            lg.sstride = lg.rep_off + (size_t)LIN_SPEC_ROWS * lg.rep_w;
        }
        const int positions = d.n_layer + 2;
        ctx->embed = o.lo == 0;
        ctx->head = o.hi == positions;
        ctx->L0 = std::max(o.lo, 1) - 1;
        ctx->L1 = std::min(o.hi, d.n_layer + 1) - 1;
        if (ctx->L1 < ctx->L0) ctx->L1 = ctx->L0;
        const int H = d.hidden, F = d.ffn, nH = d.n_heads, nKV = d.n_kv_heads, D = d.head_dim;
        // KV geometry and pool (web/model/model.js:132-147, stage.js:155-187).
        ctx->geom.nKV = nKV;
        ctx->geom.D = D;
        ctx->geom.ng = D / 32;
        ctx->geom.page = o.page_tokens;
        ctx->geom.blk = 64 * D + 64 * (D / 32) * 4;
        ctx->max_pages = ceil_div(o.n_max, o.page_tokens);
        ctx->geom.max_pages = ctx->max_pages;
        ctx->n_pages = o.slots * ctx->max_pages;
        ctx->owned.assign(o.sessions, 0);
        HIPCHK(dalloc(ctx, &ctx->page_table, (size_t)o.sessions * ctx->max_pages * 4, &ctx->scratch_bytes));
        HIPCHK(dalloc(ctx, &ctx->free_stack, (size_t)ctx->n_pages * 4, &ctx->scratch_bytes));
        {
            // Lowest index pops first (model.js:145-146): stack[i] = n_pages-1-i.
            std::vector<uint32_t> fs(ctx->n_pages);
            for (int i = 0; i < ctx->n_pages; i++) fs[i] = (uint32_t)(ctx->n_pages - 1 - i);
            HIPCHK(hipMemcpyAsync(ctx->free_stack, fs.data(), fs.size() * 4, hipMemcpyHostToDevice, ctx->stream));
            HIPCHK(hipStreamSynchronize(ctx->stream));
            ctx->top = ctx->n_pages;
        }
        const size_t pool_bytes = (size_t)ctx->n_pages * nKV * ctx->geom.blk;
        ctx->layers.resize(ctx->L1 - ctx->L0);
        bool any_full = false, any_linear = false;
        const LinGeom& lg = ctx->lg;
        for (int li = 0; li < (int)ctx->layers.size(); li++) {
            Layer& L = ctx->layers[li];
            L.kind = ctx->kinds[ctx->L0 + li];
            if (L.kind == CC_LINEAR_ATTENTION) {
                any_linear = true;
                HIPCHK(alloc_q(ctx, L.lin, lg.N, H));
                HIPCHK(alloc_q(ctx, L.out, H, lg.valueDim));
                HIPCHK(dalloc(ctx, &L.conv, (size_t)lg.convDim * LIN_CONV_K * 4, &ctx->weight_bytes));
                HIPCHK(dalloc(ctx, &L.gp, (size_t)2 * lg.nV * 4, &ctx->weight_bytes));
                HIPCHK(dalloc(ctx, &L.gnorm, (size_t)lg.Dv * 4, &ctx->weight_bytes));
                launch_fill(ctx->stream, L.gnorm, lg.Dv, 1.0f);
                // recurrent state, one block per session frame (model.js:46-58)
                HIPCHK(dalloc(ctx, &L.state, (size_t)o.sessions * lg.sstride * 4, &ctx->kv_bytes));
            } else {
                any_full = true;
                // q | k | v, and on a hybrid checkpoint the output gate's rows after v
                HIPCHK(alloc_q(ctx, L.qkv, (nH + 2 * nKV) * D + (ctx->hybrid ? nH * D : 0), H));
                HIPCHK(alloc_q(ctx, L.o, H, nH * D));
                if (ctx->hybrid) {
                    HIPCHK(dalloc(ctx, &L.qn, (size_t)D * 4, &ctx->weight_bytes));
                    HIPCHK(dalloc(ctx, &L.kn, (size_t)D * 4, &ctx->weight_bytes));
                    launch_fill(ctx->stream, L.qn, D, 1.0f);
                    launch_fill(ctx->stream, L.kn, D, 1.0f);
                }
                HIPCHK(dalloc(ctx, &L.kpool, pool_bytes, &ctx->kv_bytes));
                HIPCHK(dalloc(ctx, &L.vpool, pool_bytes, &ctx->kv_bytes));
            }
            HIPCHK(alloc_q(ctx, L.gu, 2 * F, H));
            HIPCHK(alloc_q(ctx, L.down, H, F));
            HIPCHK(dalloc(ctx, &L.ln1, (size_t)H * 4, &ctx->weight_bytes));
            HIPCHK(dalloc(ctx, &L.ln2, (size_t)H * 4, &ctx->weight_bytes));
            launch_fill(ctx->stream, L.ln1, H, 1.0f);
            launch_fill(ctx->stream, L.ln2, H, 1.0f);
        }
        (void)any_full;
        if (ctx->embed || (ctx->head && d.tied)) HIPCHK(alloc_q(ctx, ctx->wte, d.vocab, H));
        if (ctx->head) {
            HIPCHK(dalloc(ctx, &ctx->norm, (size_t)H * 4, &ctx->weight_bytes));
            launch_fill(ctx->stream, ctx->norm, H, 1.0f);
            if (!d.tied) HIPCHK(alloc_q(ctx, ctx->lm_head, d.vocab, H));
        }
        // RoPE table for every position a frame can reach.
        ctx->tbl_cap = ctx->max_pages * o.page_tokens + 64;
        {
            std::vector<float> t;
            build_rope_table(ctx, t);
            HIPCHK(dalloc(ctx, &ctx->tbl, t.size() * 4, &ctx->scratch_bytes));
            HIPCHK(hipMemcpyAsync(ctx->tbl, t.data(), t.size() * 4, hipMemcpyHostToDevice, ctx->stream));
            HIPCHK(hipStreamSynchronize(ctx->stream));
        }
        // Scratch for t_max rows.
        const int T = o.t_max;
        ctx->mt_alloc = 2 * ceil_div(T, 32);
        auto xp_bytes = [&](int K) { return (size_t)ctx->mt_alloc * 2 * ceil_div(K, 64) * 2 * 1024; };
        HIPCHK(dalloc(ctx, &ctx->x, (size_t)T * H * 4, &ctx->scratch_bytes));
        HIPCHK(dalloc(ctx, &ctx->xp_h, xp_bytes(H), &ctx->scratch_bytes));
        HIPCHK(dalloc(ctx, &ctx->xp_o, xp_bytes(nH * D), &ctx->scratch_bytes));
        HIPCHK(dalloc(ctx, &ctx->xp_f, xp_bytes(F), &ctx->scratch_bytes));
        HIPCHK(dalloc(ctx, &ctx->ssp, (size_t)16 * ctx->mt_alloc * RW_SMAX * 4, &ctx->scratch_bytes));
        if (any_linear) {
            HIPCHK(dalloc(ctx, &ctx->xp_v, xp_bytes(lg.valueDim), &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->lraw, (size_t)T * lg.W * 4, &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->lcore, (size_t)T * lg.valueDim * 4, &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->lrep, (size_t)o.max_jobs * LIN_SPEC_ROWS * lg.lrep_w * 4, &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->lring, (size_t)o.max_jobs * (LIN_CONV_K - 1) * lg.convDim * 4, &ctx->scratch_bytes));
        }
        ctx->any_linear = any_linear;
        ctx->spec_base.assign(o.sessions, 0);
        ctx->spec_n.assign(o.sessions, -1);
        ctx->fed.assign(o.sessions, 0);
        if (ctx->hybrid) HIPCHK(dalloc(ctx, &ctx->gbuf, (size_t)T * nH * D * 4, &ctx->scratch_bytes));
        size_t pf = 16;
        for (const Layer& L : ctx->layers)
            for (const QTensor* q : {&L.qkv, &L.o, &L.gu, &L.down, &L.lin, &L.out})
                if (q->codes) pf = std::max(pf, (size_t)q->P * T * q->N);
        ctx->part_floats = pf;
        HIPCHK(dalloc(ctx, &ctx->part, pf * 4, &ctx->scratch_bytes));
        // Q operands: sum over jobs of nKV * ceil(n*group/16) * ng * 2 * 64 uint4.
        ctx->qp_units = (size_t)(ceil_div(T * ctx->group, 16) + o.max_jobs) * nKV * (D / 32) * 128;
        HIPCHK(dalloc(ctx, &ctx->qp, ctx->qp_units * 16, &ctx->scratch_bytes));
        // Attention work items: `ppw` pages each, at most COMBINE_CMAX chunks a
        // frame (the combine kernel's LDS). Fixed for the context, so a row's
        // sums depend on its own chunks only. Narrow K/V rows (nKV * D <= 512,
        // SmolLM2's 3 x 64) make short items, and such a model's passes hold
        // few of them: PPW_NARROW pages an item gives more waves at the same
        // share of partial traffic.
        ctx->ppw = std::max(nKV * D <= 512 ? PPW_NARROW : 8, ceil_div(ctx->max_pages, 512));   // <= 64 (check_dims)
        ctx->items_cap = max_items_for(ctx);
        // Attention partials: 16 rows of (D + 4) floats per item.
        ctx->apart_floats = ctx->items_cap * 16 * (size_t)(D + 4);
        HIPCHK(dalloc(ctx, &ctx->apart, ctx->apart_floats * 4, &ctx->scratch_bytes));
        if (ctx->head && d.mtp_vocab > 0) {
            // the MTP head (stage.js:273-289 attachMtp): its block's KV is laid
            // out as a pool layer, addressed by each session's page table
            ctx->mtp = true;
            Layer& M = ctx->mtpL;
            HIPCHK(alloc_q(ctx, M.qkv, (nH + 2 * nKV) * D + (ctx->hybrid ? nH * D : 0), H));
            HIPCHK(alloc_q(ctx, M.o, H, nH * D));
            HIPCHK(alloc_q(ctx, M.gu, 2 * F, H));
            HIPCHK(alloc_q(ctx, M.down, H, F));
            for (float** w : {&M.ln1, &M.ln2}) {
                HIPCHK(dalloc(ctx, w, (size_t)H * 4, &ctx->weight_bytes));
                launch_fill(ctx->stream, *w, H, 1.0f);
            }
            if (ctx->hybrid) {
                for (float** w : {&M.qn, &M.kn}) {
                    HIPCHK(dalloc(ctx, w, (size_t)D * 4, &ctx->weight_bytes));
                    launch_fill(ctx->stream, *w, D, 1.0f);
                }
            }
            HIPCHK(dalloc(ctx, &M.kpool, pool_bytes, &ctx->kv_bytes));
            HIPCHK(dalloc(ctx, &M.vpool, pool_bytes, &ctx->kv_bytes));
            HIPCHK(alloc_q(ctx, ctx->fc_e, H, H));
            HIPCHK(alloc_q(ctx, ctx->fc_h, H, H));
            HIPCHK(alloc_q(ctx, ctx->embed_draft, d.mtp_vocab, H));
            HIPCHK(alloc_q(ctx, ctx->head_draft, d.mtp_vocab, H));
            for (float** w : {&ctx->enorm, &ctx->hnorm, &ctx->mtp_norm}) {
                HIPCHK(dalloc(ctx, w, (size_t)H * 4, &ctx->weight_bytes));
                launch_fill(ctx->stream, *w, H, 1.0f);
            }
            HIPCHK(dalloc(ctx, &ctx->mtpH, (size_t)o.sessions * H * 4, &ctx->scratch_bytes));
            for (float** b : {&ctx->mx, &ctx->mtp_in, &ctx->mtp_e})
                HIPCHK(dalloc(ctx, b, (size_t)T * H * 4, &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->xp_e, xp_bytes(H), &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->xp_hh, xp_bytes(H), &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->mtp_logits, (size_t)ctx->head_draft.P * d.mtp_vocab * 4, &ctx->scratch_bytes));
            // one region per draft step: a one-row job's plan
            const size_t mtq1 = ceil_div(ctx->group, 16);
            const size_t a256 = 255;
            auto al = [&](size_t b) { return (b + a256) & ~a256; };
            ctx->chain_step = al(sizeof(JobDev)) + al(sizeof(AttnItem) * nKV * mtq1 * ceil_div(ctx->max_pages, ctx->ppw)) +
                              al(4) + al(12 * nKV * mtq1);
            const size_t cb = 256 + MTP_STEPS_MAX * ctx->chain_step;
            HIPCHK(dalloc(ctx, &ctx->d_chain, cb, &ctx->scratch_bytes));
            HIPCHK(hipHostMalloc((void**)&ctx->h_chain, cb, hipHostMallocDefault));
        }
        if (ctx->head) {
            ctx->head_planes = lx_planes_for(d.vocab, H, ctx->ncu);   // the head tensor's own planes
            HIPCHK(dalloc(ctx, &ctx->logits, (size_t)ctx->head_planes * T * d.vocab * 4, &ctx->scratch_bytes));
            const size_t keys = (size_t)T * ceil_div(d.vocab, 4096) * TOPK_MAX;
            HIPCHK(dalloc(ctx, &ctx->tk_a, keys * 8, &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->tk_b, keys * 8, &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->d_vals, (size_t)T * TOPK_MAX * 4, &ctx->scratch_bytes));
            HIPCHK(dalloc(ctx, &ctx->d_ids, (size_t)T * TOPK_MAX * 4, &ctx->scratch_bytes));
        }
        HIPCHK(dalloc(ctx, &ctx->d_hbits, (size_t)T * H * 2, &ctx->scratch_bytes));
        MetaLayout ml = meta_layout(ctx);
        ctx->meta_bytes = ml.total;
        HIPCHK(dalloc(ctx, &ctx->d_meta, ml.total, &ctx->scratch_bytes));
        HIPCHK(hipHostMalloc((void**)&ctx->h_meta, ml.total, hipHostMallocDefault));
        ctx->out_bytes = std::max((size_t)T * TOPK_MAX * 8, (size_t)T * H * 2) + 256;
        HIPCHK(hipHostMalloc(&ctx->h_out, ctx->out_bytes, hipHostMallocDefault));
        HIPCHK(hipStreamSynchronize(ctx->stream));
        return CC_OK;
    };
    st = body();
    *out = ctx;
    return st;
}

static QTensor* tensor_of(cc_ctx* ctx, int layer, int tensor, int* row_tile0, int* N, int* K) {
    const cc_dims& d = ctx->d;
    const int H = d.hidden, F = d.ffn, D = d.head_dim, nH = d.n_heads, nKV = d.n_kv_heads;
    if (tensor == CC_T_WTE) { *row_tile0 = 0; *N = d.vocab; *K = H; return ctx->wte.codes ? &ctx->wte : nullptr; }
    if (tensor == CC_T_LM_HEAD) { *row_tile0 = 0; *N = d.vocab; *K = H; return ctx->lm_head.codes ? &ctx->lm_head : nullptr; }
    if (tensor >= CC_T_MTP_FC_E && tensor <= CC_T_MTP_HEAD) {
        if (!ctx->mtp) return nullptr;
        *row_tile0 = 0;
        *K = H;
        *N = tensor == CC_T_MTP_FC_E || tensor == CC_T_MTP_FC_H ? H : d.mtp_vocab;
        switch (tensor) {
            case CC_T_MTP_FC_E: return &ctx->fc_e;
            case CC_T_MTP_FC_H: return &ctx->fc_h;
            case CC_T_MTP_EMBED: return &ctx->embed_draft;
            case CC_T_MTP_HEAD: return &ctx->head_draft;
        }
        return nullptr;
    }
    Layer* Lp = nullptr;
    if (layer == CC_LAYER_MTP) {
        if (ctx->mtp) Lp = &ctx->mtpL;
    } else {
        const int li = layer - ctx->L0;
        if (li >= 0 && li < (int)ctx->layers.size()) Lp = &ctx->layers[li];
    }
    if (!Lp) return nullptr;
    Layer& L = *Lp;
    if (L.kind == CC_LINEAR_ATTENTION) {
        // fused in_proj rows: q | k | v | z | b (nVp) | a (nVp)
        const LinGeom& lg = ctx->lg;
        const int kd = lg.keyDim, vd = lg.valueDim;
        switch (tensor) {
            case CC_T_IN_Q: *row_tile0 = 0; *N = kd; *K = H; return &L.lin;
            case CC_T_IN_K: *row_tile0 = kd / 16; *N = kd; *K = H; return &L.lin;
            case CC_T_IN_V: *row_tile0 = 2 * kd / 16; *N = vd; *K = H; return &L.lin;
            case CC_T_IN_Z: *row_tile0 = (2 * kd + vd) / 16; *N = vd; *K = H; return &L.lin;
            case CC_T_IN_B: *row_tile0 = (2 * kd + 2 * vd) / 16; *N = lg.nV; *K = H; return &L.lin;
            case CC_T_IN_A: *row_tile0 = (2 * kd + 2 * vd + lg.nVp) / 16; *N = lg.nV; *K = H; return &L.lin;
            case CC_T_OUT_PROJ: *row_tile0 = 0; *N = H; *K = vd; return &L.out;
            case CC_T_GATE: *row_tile0 = 0; *N = F; *K = H; return &L.gu;
            case CC_T_UP: *row_tile0 = F / 16; *N = F; *K = H; return &L.gu;
            case CC_T_DOWN: *row_tile0 = 0; *N = H; *K = F; return &L.down;
        }
        return nullptr;
    }
    switch (tensor) {
        case CC_T_ATTN_GATE:
            if (!ctx->hybrid) return nullptr;
            *row_tile0 = (nH + 2 * nKV) * D / 16; *N = nH * D; *K = H; return &L.qkv;
        case CC_T_Q: *row_tile0 = 0; *N = nH * D; *K = H; return &L.qkv;
        case CC_T_K: *row_tile0 = nH * D / 16; *N = nKV * D; *K = H; return &L.qkv;
        case CC_T_V: *row_tile0 = (nH + nKV) * D / 16; *N = nKV * D; *K = H; return &L.qkv;
        case CC_T_O: *row_tile0 = 0; *N = H; *K = nH * D; return &L.o;
        case CC_T_GATE: *row_tile0 = 0; *N = F; *K = H; return &L.gu;
        case CC_T_UP: *row_tile0 = F / 16; *N = F; *K = H; return &L.gu;
        case CC_T_DOWN: *row_tile0 = 0; *N = H; *K = F; return &L.down;
    }
    return nullptr;
}

cc_status cc_upload(cc_ctx* ctx, int32_t layer, int32_t tensor, const void* data, size_t n, const void* scales,
                    size_t ns, int32_t scale_dtype, int32_t group) {
    if (!ctx || !data) return fail(ctx, CC_EARG, "null argument");
    const cc_dims& d = ctx->d;
    const bool f32_tensor = tensor == CC_T_LN1 || tensor == CC_T_LN2 || tensor == CC_T_NORM ||
                            (tensor >= CC_T_Q_NORM && tensor <= CC_T_K_NORM) ||
                            (tensor >= CC_T_CONV_Q && tensor <= CC_T_GATED_NORM) || tensor == CC_T_MTP_ENORM ||
                            tensor == CC_T_MTP_HNORM || tensor == CC_T_MTP_NORM;
    if (f32_tensor) {
        float* dst = nullptr;
        size_t want = d.hidden;
        if (tensor == CC_T_NORM) dst = ctx->norm;
        else if (tensor == CC_T_MTP_ENORM) dst = ctx->enorm;
        else if (tensor == CC_T_MTP_HNORM) dst = ctx->hnorm;
        else if (tensor == CC_T_MTP_NORM) dst = ctx->mtp_norm;
        else {
            const int li = layer - ctx->L0;
            const bool m = layer == CC_LAYER_MTP && ctx->mtp;
            if (!m && (li < 0 || li >= (int)ctx->layers.size())) return fail(ctx, CC_EARG, "layer not held here");
            Layer& L = m ? ctx->mtpL : ctx->layers[li];
            const LinGeom& lg = ctx->lg;
            switch (tensor) {
                case CC_T_LN1: dst = L.ln1; break;
                case CC_T_LN2: dst = L.ln2; break;
                case CC_T_Q_NORM: dst = L.qn; want = d.head_dim; break;
                case CC_T_K_NORM: dst = L.kn; want = d.head_dim; break;
                // conv weights [channels][4], the q, k, v channel ranges in order
                case CC_T_CONV_Q: dst = L.conv; want = (size_t)lg.keyDim * LIN_CONV_K; break;
                case CC_T_CONV_K:
                    dst = L.conv ? L.conv + (size_t)lg.keyDim * LIN_CONV_K : nullptr;
                    want = (size_t)lg.keyDim * LIN_CONV_K;
                    break;
                case CC_T_CONV_V:
                    dst = L.conv ? L.conv + (size_t)2 * lg.keyDim * LIN_CONV_K : nullptr;
                    want = (size_t)lg.valueDim * LIN_CONV_K;
                    break;
                case CC_T_GATE_PARAMS: dst = L.gp; want = (size_t)2 * lg.nV; break;
                case CC_T_GATED_NORM: dst = L.gnorm; want = lg.Dv; break;
            }
        }
        if (!dst) return fail(ctx, CC_EARG, "tensor not held here");
        if (n != want)
            return fail(ctx, CC_EARG, "f32 tensor " + std::to_string(tensor) + " has " + std::to_string(want) +
                                          " values, not " + std::to_string(n));
        HIPCHK(hipMemcpyAsync(dst, data, n * 4, hipMemcpyHostToDevice, ctx->stream));
        HIPCHK(hipStreamSynchronize(ctx->stream));
        return CC_OK;
    }
    int row_tile0 = 0, N = 0, K = 0;
    QTensor* q = tensor_of(ctx, layer, tensor, &row_tile0, &N, &K);
    if (!q) return fail(ctx, CC_EARG, "tensor not held here");
    if (group < 32 || group % 32) return fail(ctx, CC_EARG, "q8 group must be a multiple of 32");
    const int ngi = ceil_div(K, group);
    if (n != (size_t)N * K || ns != (size_t)N * ngi || !scales)
        return fail(ctx, CC_EARG, "q8 tensor needs N*K codes and N*ceil(K/group) scales");
    // f32 scales of a group of 64 or a multiple (the converter's, loaded by
    // uploadQ8, web/model/kernels.js:116-126) stay f32: one per row and
    // 64-wide unit, in the same bytes f16 scales per 32 take. Other groups
    // keep one f16 scale per 32 values (f32 ones rounded to it). A wider
    // group's scale repeats over its units or groups, exactly.
    const bool f32u = scale_dtype == CC_SCALES_F32 && group % 64 == 0;
    if (f32u ? q->up_f16 : q->up_f32)
        return fail(ctx, CC_EARG, "the parts of a fused q8 tensor need one scale format: f32 scales with a group "
                                  "of 64 (or a multiple) for every part, or none");
    std::vector<uint8_t> sv;
    if (f32u) {
        const int rep = group / 64;
        sv.resize((size_t)N * q->KU * 4);
        float* s32 = (float*)sv.data();
        for (size_t row = 0; row < (size_t)N; row++)
            for (int u = 0; u < q->KU; u++) s32[row * q->KU + u] = ((const float*)scales)[row * ngi + u / rep];
    } else {
        const int ng = ceil_div(K, 32), rep = group / 32;
        sv.resize((size_t)N * ng * 2);
        uint16_t* s16 = (uint16_t*)sv.data();
        for (size_t row = 0; row < (size_t)N; row++)
            for (int g = 0; g < ng; g++) {
                const size_t i = row * ngi + g / rep;
                s16[row * ng + g] = scale_dtype == CC_SCALES_F16 ? ((const uint16_t*)scales)[i]
                                                                 : half_bits(((const float*)scales)[i]);
            }
    }
    q->f32s = f32u ? 1 : 0;
    (f32u ? q->up_f32 : q->up_f16)++;
    int8_t* dc = nullptr;
    uint8_t* ds = nullptr;
    HIPCHK(hipMalloc(&dc, n));
    HIPCHK(hipMalloc(&ds, sv.size()));
    HIPCHK(hipMemcpy(dc, data, n, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(ds, sv.data(), sv.size(), hipMemcpyHostToDevice));
    launch_tile_q8(ctx->stream, dc, ds, N, K, *q, row_tile0);
    HIPCHK(hipStreamSynchronize(ctx->stream));
    (void)hipFree(dc);
    (void)hipFree(ds);
    return CC_OK;
}

// Generator streams shared with the test oracle: wte 1, lm_head 2, block
// tensor t of layer l: (l+1)*16 + t (q, k, v, o, gate, up, down).
// Every q8 tensor of the context back to f16 scales per 32 with no parts
// uploaded (the synthetic fill writes that format everywhere).
static void reset_scale_formats(cc_ctx* ctx) {
    auto reset = [](QTensor& q) { q.f32s = q.up_f16 = q.up_f32 = 0; };
    for (Layer& L : ctx->layers)
        for (QTensor* q : {&L.qkv, &L.o, &L.gu, &L.down, &L.lin, &L.out}) reset(*q);
    for (QTensor* q : {&ctx->mtpL.qkv, &ctx->mtpL.o, &ctx->mtpL.gu, &ctx->mtpL.down, &ctx->fc_e, &ctx->fc_h,
                       &ctx->embed_draft, &ctx->head_draft, &ctx->wte, &ctx->lm_head})
        reset(*q);
}

cc_status cc_fill_random(cc_ctx* ctx, uint64_t seed) {
    if (!ctx) return CC_EARG;
    const cc_dims& d = ctx->d;
    hipStream_t st = ctx->stream;
    reset_scale_formats(ctx);
    for (int li = 0; li < (int)ctx->layers.size(); li++) {
        const int layer = ctx->L0 + li;
        Layer& L = ctx->layers[li];
        if (L.kind == CC_LINEAR_ATTENTION) {
            // synthetic Gated DeltaNet weights (timing only; the parity tests
            // upload theirs): the fused in_proj and out_proj from the
            // generator, fixed conv taps and gates
            const LinGeom& lg = ctx->lg;
            launch_gen_q8(st, L.lin, 0, lg.N, d.hidden, seed, (uint64_t)(layer + 1) * 16 + 7);
            launch_gen_q8(st, L.out, 0, d.hidden, lg.valueDim, seed, (uint64_t)(layer + 1) * 16 + 8);
            launch_fill(st, L.conv, (int64_t)lg.convDim * LIN_CONV_K, 0.25f);
            launch_fill(st, L.gp, lg.nV, -1.0f);          // A_log
            launch_fill(st, L.gp + lg.nV, lg.nV, 0.0f);   // dt_bias
            for (int t = CC_T_GATE; t <= CC_T_DOWN; t++) {
                int row_tile0, N, K;
                QTensor* q = tensor_of(ctx, layer, t, &row_tile0, &N, &K);
                launch_gen_q8(st, *q, row_tile0, N, K, seed, (uint64_t)(layer + 1) * 16 + t);
            }
            continue;
        }
        for (int t = CC_T_Q; t <= CC_T_DOWN; t++) {
            int row_tile0, N, K;
            QTensor* q = tensor_of(ctx, layer, t, &row_tile0, &N, &K);
            launch_gen_q8(st, *q, row_tile0, N, K, seed, (uint64_t)(layer + 1) * 16 + t);
        }
        if (ctx->hybrid) {
            int row_tile0, N, K;
            QTensor* q = tensor_of(ctx, layer, CC_T_ATTN_GATE, &row_tile0, &N, &K);
            launch_gen_q8(st, *q, row_tile0, N, K, seed, (uint64_t)(layer + 1) * 16 + 12);
        }
    }
    if (ctx->mtp) {
        // the MTP head's matmuls and block (timing only)
        const int H = d.hidden;
        launch_gen_q8(st, ctx->fc_e, 0, H, H, seed, 3);
        launch_gen_q8(st, ctx->fc_h, 0, H, H, seed, 4);
        launch_gen_q8(st, ctx->embed_draft, 0, d.mtp_vocab, H, seed, 5);
        launch_gen_q8(st, ctx->head_draft, 0, d.mtp_vocab, H, seed, 6);
        for (int t = CC_T_Q; t <= CC_T_DOWN; t++) {
            int row_tile0, N, K;
            QTensor* q = tensor_of(ctx, CC_LAYER_MTP, t, &row_tile0, &N, &K);
            launch_gen_q8(st, *q, row_tile0, N, K, seed, 0x4D545000ull + t);
        }
    }
    if (ctx->wte.codes) launch_gen_q8(ctx->stream, ctx->wte, 0, d.vocab, d.hidden, seed, 1);
    if (ctx->lm_head.codes) launch_gen_q8(ctx->stream, ctx->lm_head, 0, d.vocab, d.hidden, seed, 2);
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return CC_OK;
}

int32_t cc_slot_pages(const cc_ctx* ctx, int32_t slot) {
    if (!ctx || slot < 0 || slot >= (int)ctx->owned.size()) return -1;
    return ctx->owned[slot];
}

int32_t cc_free_pages(const cc_ctx* ctx) { return ctx ? ctx->top : -1; }

// Takes pages for jobs (slot, tokens) in order: ensurePages replayed on the
// device. Validates capacity first; nothing changes on failure.
static cc_status take_pages(cc_ctx* ctx, const std::vector<std::pair<int, int>>& want, int32_t* d_plan,
                            int32_t* h_plan, int32_t* status) {
    int total = 0;
    for (size_t j = 0; j < want.size(); j++) {
        const int slot = want[j].first, tokens = want[j].second;
        const int need = ceil_div(tokens, ctx->geom.page);
        if (need > ctx->max_pages) {
            if (status) status[j] = CC_EPOOL;
            return fail(ctx, CC_EPOOL, "the KV pool cannot fit " + std::to_string(tokens) + " tokens for slot " +
                                           std::to_string(slot) + " (" + std::to_string(ctx->max_pages) +
                                           " pages of " + std::to_string(ctx->geom.page) + " per frame)");
        }
        const int nw = std::max(0, need - ctx->owned[slot]);
        h_plan[4 * j] = slot;
        h_plan[4 * j + 1] = ctx->owned[slot];
        h_plan[4 * j + 2] = nw;
        h_plan[4 * j + 3] = total;
        total += nw;
    }
    if (total > ctx->top) {
        if (status) for (size_t j = 0; j < want.size(); j++) status[j] = CC_BUSY;
        return fail(ctx, CC_BUSY, "no KV page free for the pass (" + std::to_string(total) + " needed, " +
                                      std::to_string(ctx->top) + " free)");
    }
    if (total > 0) {
        launch_alloc_pages(ctx->stream, d_plan, (int)want.size(), ctx->free_stack, ctx->top, ctx->page_table,
                           ctx->max_pages);
        for (size_t j = 0; j < want.size(); j++) ctx->owned[want[j].first] += h_plan[4 * j + 2];
        ctx->top -= total;
    }
    return CC_OK;
}

cc_status cc_release(cc_ctx* ctx, int32_t slot) {
    if (!ctx || slot < 0 || slot >= (int)ctx->owned.size()) return fail(ctx, CC_EARG, "bad slot");
    const int n = ctx->owned[slot];
    launch_release_pages(ctx->stream, slot, n, ctx->free_stack, ctx->top, ctx->page_table, ctx->max_pages);
    ctx->top += n;
    ctx->owned[slot] = 0;
    ctx->spec_n[slot] = -1;
    ctx->fed[slot] = 0;
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return CC_OK;
}

cc_status cc_fill_random_kv(cc_ctx* ctx, int32_t slot, int32_t tokens, uint64_t seed, uint64_t key) {
    if (!ctx || slot < 0 || slot >= (int)ctx->owned.size() || tokens < 0 || tokens > ctx->o.n_max)
        return fail(ctx, CC_EARG, "bad slot or token count");
    int32_t* h_plan = (int32_t*)ctx->h_meta;
    int32_t* d_plan = (int32_t*)ctx->d_meta;
    std::vector<std::pair<int, int>> want{{slot, tokens}};
    const int need = ceil_div(tokens, ctx->geom.page);
    if (need > ctx->max_pages) return fail(ctx, CC_EPOOL, "the fill exceeds the frame's pages");
    h_plan[0] = slot; h_plan[1] = ctx->owned[slot]; h_plan[2] = std::max(0, need - ctx->owned[slot]); h_plan[3] = 0;
    HIPCHK(hipMemcpyAsync(d_plan, h_plan, 16, hipMemcpyHostToDevice, ctx->stream));
    cc_status st = take_pages(ctx, want, d_plan, h_plan, nullptr);
    if (st != CC_OK) return st;
    for (int li = 0; li < (int)ctx->layers.size(); li++) {
        const int layer = ctx->L0 + li;
        if (!ctx->layers[li].kpool) continue;   // a linear_attention block keeps no KV
        for (int which = 0; which < 2; which++)
            launch_fill_kv(ctx->stream, which ? ctx->layers[li].vpool : ctx->layers[li].kpool, ctx->page_table,
                           slot, tokens, ctx->geom, seed, 0x4B560000ull + (uint64_t)layer * 2 + which, key, which);
    }
    // a synthetic history: the recurrent blocks hold these rows (their state
    // is whatever the session's state block holds)
    ctx->fed[slot] = tokens;
    ctx->spec_n[slot] = -1;
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return CC_OK;
}

static cc_status kv_io(cc_ctx* ctx, int32_t layer, int32_t which, int32_t slot, int32_t head, int32_t t0,
                       int32_t t1, uint32_t* out, const uint32_t* in) {
    const int li = layer - ctx->L0;
    if (li < 0 || li >= (int)ctx->layers.size() || which < 0 || which > 1 || slot < 0 ||
        slot >= (int)ctx->owned.size() || head < 0 || head >= ctx->geom.nKV || t0 < 0 || t1 < t0 ||
        ceil_div(t1, ctx->geom.page) > ctx->owned[slot])
        return fail(ctx, CC_EARG, "rows outside the slot's pages");
    if (!ctx->layers[li].kpool) return fail(ctx, CC_EARG, "a linear_attention block keeps no KV");
    const size_t words = (size_t)(t1 - t0) * (ctx->geom.D / 4 + ctx->geom.ng);
    uint32_t* dbuf = nullptr;
    HIPCHK(hipMalloc(&dbuf, words * 4 + 16));
    uint8_t* pool = which ? ctx->layers[li].vpool : ctx->layers[li].kpool;
    if (out) {
        launch_kv_to_ref(ctx->stream, pool, ctx->page_table, slot, head, t0, t1, ctx->geom, which, dbuf);
        HIPCHK(hipStreamSynchronize(ctx->stream));
        HIPCHK(hipMemcpy(out, dbuf, words * 4, hipMemcpyDeviceToHost));
    } else {
        HIPCHK(hipMemcpy(dbuf, in, words * 4, hipMemcpyHostToDevice));
        launch_kv_from_ref(ctx->stream, pool, ctx->page_table, slot, head, t0, t1, ctx->geom, which, dbuf);
        HIPCHK(hipStreamSynchronize(ctx->stream));
    }
    (void)hipFree(dbuf);
    return CC_OK;
}

cc_status cc_read_kv(cc_ctx* ctx, int32_t layer, int32_t which, int32_t slot, int32_t head, int32_t t0,
                     int32_t t1, uint32_t* out) {
    if (!ctx || !out) return CC_EARG;
    return kv_io(ctx, layer, which, slot, head, t0, t1, out, nullptr);
}

cc_status cc_write_kv(cc_ctx* ctx, int32_t layer, int32_t which, int32_t slot, int32_t head, int32_t t0,
                      int32_t t1, const uint32_t* rows) {
    if (!ctx || !rows) return CC_EARG;
    return kv_io(ctx, layer, which, slot, head, t0, t1, nullptr, rows);
}

cc_status cc_read_pages(cc_ctx* ctx, int32_t slot, uint32_t* out, int32_t n) {
    if (!ctx || !out || slot < 0 || slot >= (int)ctx->owned.size() || n < 0 || n > ctx->max_pages)
        return fail(ctx, CC_EARG, "bad slot or count");
    HIPCHK(hipStreamSynchronize(ctx->stream));
    HIPCHK(hipMemcpy(out, ctx->page_table + (size_t)slot * ctx->max_pages, (size_t)n * 4, hipMemcpyDeviceToHost));
    return CC_OK;
}

cc_status cc_read_logits(cc_ctx* ctx, int32_t rows, float* out) {
    if (!ctx || !out || !ctx->logits || rows < 1 || rows != ctx->head_rows)
        return fail(ctx, CC_EARG, "rows must be the last pass's sampled rows");
    HIPCHK(hipStreamSynchronize(ctx->stream));
    // The head's planes, added in plane order as the sampling kernels add them.
    const size_t n = (size_t)rows * ctx->d.vocab;
    std::vector<float> plane(n);
    HIPCHK(hipMemcpy(out, ctx->logits, n * 4, hipMemcpyDeviceToHost));
    const int planes = gemm_planes(ctx->d.tied ? ctx->wte : ctx->lm_head, rows, ctx->ncu);
    for (int q = 1; q < planes; q++) {
        HIPCHK(hipMemcpy(plane.data(), ctx->logits + q * n, n * 4, hipMemcpyDeviceToHost));
        for (size_t i = 0; i < n; i++) out[i] = out[i] + plane[i];
    }
    return CC_OK;
}

cc_status cc_stats_get(const cc_ctx* ctx, cc_stats* out) {
    if (!ctx || !out) return CC_EARG;
    out->weight_bytes = ctx->weight_bytes;
    out->kv_bytes = ctx->kv_bytes;
    out->scratch_bytes = ctx->scratch_bytes;
    out->vram_bytes = ctx->weight_bytes + ctx->kv_bytes + ctx->scratch_bytes;
    out->passes = ctx->passes;
    out->rows = ctx->rows;
    out->last_pass_ms = ctx->last_ms;
    return CC_OK;
}

cc_status cc_profile(cc_ctx* ctx, int32_t enable) {
    if (!ctx) return CC_EARG;
    ctx->prof = enable != 0;
    for (int k = 0; k < CC_K_COUNT; k++) { ctx->prof_ms[k] = 0; ctx->prof_n[k] = 0; ctx->prof_bytes[k] = 0; }
    ctx->marks.clear();
    return CC_OK;
}

cc_status cc_profile_read(const cc_ctx* ctx, int32_t kind, double* ms, int64_t* launches, double* bytes) {
    if (!ctx || kind < 0 || kind >= CC_K_COUNT) return CC_EARG;
    if (ms) *ms = ctx->prof_ms[kind];
    if (launches) *launches = ctx->prof_n[kind];
    if (bytes) *bytes = ctx->prof_bytes[kind];
    return CC_OK;
}

// The step plan (stage.js:1319-1325): the per-job table with rows packed in
// job order, and the pass's counts (rows, sampled rows, attention work
// items, combine triples, Q operand and partial sizes). Work item counts:
// per (kv head, m-tile) one per chunk of ppw pages; k_pack writes the same
// tables on the device, plan_tables on the host.
static void plan_jobs(cc_ctx* ctx, const cc_job* jobs, int njobs, StepPlan& p, bool head) {
    p.jobs.resize(njobs);
    p.kv_bytes = 0;
    const int ng = ctx->geom.ng;
    size_t qp = 0;
    int row = 0, items = 0, cwg = 0, S = 0, nlaunch = 0;
    p.multi = 0;
    for (int j = 0; j < njobs; j++) {
        JobDev& jd = p.jobs[j];
        jd.slot = jobs[j].slot;
        jd.past = jobs[j].past;
        jd.n = jobs[j].n;
        jd.row0 = row;
        jd.mtq = ceil_div(jd.n * ctx->group, 16);
        jd.snap = jobs[j].snap ? 1 : 0;
        jd.keep = jobs[j].rollback ? jobs[j].keep : -1;
        jd.qp_off = (int32_t)qp;
        qp += (size_t)ctx->geom.nKV * jd.mtq * ng * 128;
        const int T_act = jd.past + jd.n;
        p.kv_bytes += 2.0 * T_act * ctx->geom.nKV * (ctx->D + 4.0 * ctx->geom.ng);
        jd.nchunk = ceil_div(ceil_div(T_act, ctx->geom.page), ctx->ppw);
        jd.item0 = items;
        items += ctx->geom.nKV * jd.mtq * jd.nchunk;
        nlaunch += ctx->geom.nKV * jd.nchunk * (jd.mtq > 1 ? 4 * ceil_div(jd.mtq, 4) : 1);
        cwg += ctx->geom.nKV * jd.mtq;
        if (jd.mtq > 1) p.multi = 1;
        if (head) S += jobs[j].sampled;
        row += jd.n;
    }
    p.T = row;
    p.S = S;
    p.nitems = items;
    p.nlaunch = nlaunch;
    p.ncwg = cwg;
    p.qp_units = qp;
    p.apart_floats = (size_t)items * 16 * (ctx->D + 4);
}

// The pass's tables on the host, for the passes that upload them (the MTP
// draft chain, the kernel-level ops).
static void plan_tables(cc_ctx* ctx, const cc_job* jobs, int njobs, StepPlan& p, bool head) {
    p.items.clear();
    p.row_job.clear();
    p.head_rows.clear();
    p.cwg.clear();
    const int ng = ctx->geom.ng, part = 16 * (ctx->D + 4);
    // k_pack's order: the jobs of several m-tiles as (kv head, chunk, block of
    // 4 m-tiles) workgroups, then the jobs of one m-tile, their full chunks
    // (pass 1) before their short last chunks (pass 2)
    for (int pass = 0; pass < 3; pass++)
        for (int j = 0; j < njobs; j++) {
            const JobDev& jd = p.jobs[j];
            if ((jd.mtq > 1) != (pass == 0)) continue;
            const int nb = jd.mtq > 1 ? ceil_div(jd.mtq, 4) : 1, per = jd.mtq > 1 ? 4 : 1;
            const int nfull = ceil_div(jd.past + jd.n, ctx->geom.page) / ctx->ppw;
            const int c0 = pass == 2 ? nfull : 0, c1 = pass == 1 ? nfull : jd.nchunk;
            for (int h = 0; h < ctx->geom.nKV; h++)
                for (int c = c0; c < c1; c++)
                    for (int b = 0; b < nb; b++)
                        for (int q = 0; q < per; q++) {
                            const int mt = per * b + q;
                            if (mt >= jd.mtq) {
                                p.items.push_back(AttnItem{0, 0, 0, -1, 0, 0, 0, 0});
                                continue;
                            }
                            const int hm = h * jd.mtq + mt;
                            const int32_t idx = jd.item0 + hm * jd.nchunk + c;
                            p.items.push_back(AttnItem{jd.slot, jd.past, jd.n, mt, jd.qp_off + hm * ng * 128,
                                                       idx * part, h, c * ctx->ppw});
                        }
        }
    for (int j = 0; j < njobs; j++) {
        const JobDev& jd = p.jobs[j];
        for (int h = 0; h < ctx->geom.nKV; h++)
            for (int mt = 0; mt < jd.mtq; mt++) {
                p.cwg.push_back(j);
                p.cwg.push_back(h);
                p.cwg.push_back(mt);
            }
        for (int i = 0; i < jd.n; i++) p.row_job.push_back(j);
        if (head)
            for (int i = jd.n - jobs[j].sampled; i < jd.n; i++) p.head_rows.push_back(jd.row0 + i);
    }
}

static void build_plan(cc_ctx* ctx, const cc_job* jobs, int njobs, StepPlan& p, bool head) {
    plan_jobs(ctx, jobs, njobs, p, head);
    plan_tables(ctx, jobs, njobs, p, head);
}

static cc_status grow(cc_ctx* ctx, const StepPlan& p) {
    if (p.qp_units > ctx->qp_units) {
        uint4* q = nullptr;
        HIPCHK(dfree(ctx, ctx->qp, ctx->qp_units * 16, &ctx->scratch_bytes));
        ctx->qp = nullptr;
        ctx->qp_units = 0;
        HIPCHK(dalloc(ctx, &q, p.qp_units * 16, &ctx->scratch_bytes));
        ctx->qp = q;
        ctx->qp_units = p.qp_units;
    }
    if (p.apart_floats > ctx->apart_floats) {
        float* a = nullptr;
        HIPCHK(dfree(ctx, ctx->apart, ctx->apart_floats * 4, &ctx->scratch_bytes));
        ctx->apart = nullptr;
        ctx->apart_floats = 0;
        HIPCHK(dalloc(ctx, &a, p.apart_floats * 4, &ctx->scratch_bytes));
        ctx->apart = a;
        ctx->apart_floats = p.apart_floats;
    }
    return CC_OK;
}

// The blocks [p0, p1) (model indices) over the packed rows: blockSegs
// (web/model/model.js:619-624) per layer, with the reference's dispatches
// fused into: operand prep, q|k|v GEMM, finish (rmsnorm's row factor + RoPE +
// KV store + Q operand), attention, combine (o_proj operand), o GEMM,
// residual (+ operand x*ln2 and the row's sum of squares), gate|up GEMM,
// finish (row factor + SwiGLU), down GEMM, residual (+ round_f16 + the next
// block's operand x*ln1 and sum of squares).
// Device pointers of a pass's metadata, and its counts.
struct PassMeta {
    const JobDev* jobs = nullptr;
    const AttnItem* items = nullptr;
    const int32_t* row_job = nullptr;
    const int32_t* cwg = nullptr;
    int njobs = 0, nitems = 0, ncwg = 0, nlaunch = 0, multi = 0;
};

static RowScale row_scale_of(const cc_ctx* ctx) {
    RowScale rs;
    rs.ssp = ctx->ssp;
    rs.nsl = ceil_div(ctx->d.hidden / 4, RW_THREADS);
    rs.H = ctx->d.hidden;
    rs.eps = ctx->d.rms_eps;
    return rs;
}

// fullBlockSegs's attention half (model.js:368-410) on rows x [T][H] whose
// operand x*ln1 and sums of squares are in place: q|k|v (+ attn_gate) GEMM,
// finish (row factor, q/k norm, RoPE, KV store, Q operand), attention,
// combine (output gate, o_proj operand), o GEMM, residual with the operand
// x*ln2 for the MLP.
static void full_attn_half(cc_ctx* ctx, Layer& L, float* x, int T, int Mpad, const PassMeta& pm) {
    const cc_dims& d = ctx->d;
    hipStream_t st = ctx->stream;
    const int H = d.hidden, nH = d.n_heads;
    const RowScale rs = row_scale_of(ctx);
    QkExtras ex;
    if (ctx->hybrid) {
        ex.qn = L.qn;
        ex.kn = L.kn;
        ex.eps = d.rms_eps;
        ex.gate = ctx->gbuf;
    }
    launch_gemm(st, L.qkv, ctx->xp_h, ctx->mt_alloc, ctx->part, T, ctx->ncu);
    launch_fin_qkv(st, ctx->part, gemm_planes(L.qkv, T, ctx->ncu), T, pm.row_job, pm.jobs, nH, ctx->group, ctx->geom, ctx->tbl, ctx->rot,
                   L.kpool, L.vpool, ctx->page_table, ctx->qp, rs, 1, 1, ex);
    launch_attn(st, pm.items, pm.nlaunch, ctx->qp, L.kpool, L.vpool, ctx->page_table, ctx->geom, ctx->group,
                ctx->ppw, ctx->apart, pm.multi, ctx->attn);
    launch_attn_combine(st, pm.jobs, ctx->apart, ctx->geom, nH, ctx->group, L.o.KU, ctx->xp_o, nullptr, pm.cwg,
                        pm.ncwg, ctx->hybrid ? ctx->gbuf : nullptr);
    launch_gemm(st, L.o, ctx->xp_o, ctx->mt_alloc, ctx->part, T, ctx->ncu);
    launch_resid_w(st, x, ctx->part, gemm_planes(L.o, T, ctx->ncu), T, Mpad, H, 0, L.ln2, ceil_div(H, 64), ctx->xp_h, ctx->ssp);
}

// The SwiGLU MLP (model.js:307-315) from the operand x*ln2: gate|up GEMM,
// finish (row factor, silu*up), down GEMM, residual (+ round_f16 for a
// trunk block) and the next block's operand x*next_ln1 (or none).
static void ffn_half(cc_ctx* ctx, Layer& L, float* x, int T, int Mpad, int round, const float* next_ln1) {
    const cc_dims& d = ctx->d;
    hipStream_t st = ctx->stream;
    const int H = d.hidden;
    const RowScale rs = row_scale_of(ctx);
    launch_gemm(st, L.gu, ctx->xp_h, ctx->mt_alloc, ctx->part, T, ctx->ncu);
    launch_fin_swiglu(st, ctx->part, gemm_planes(L.gu, T, ctx->ncu), T, Mpad, d.ffn, L.down.KU, ctx->xp_f, rs);
    launch_gemm(st, L.down, ctx->xp_f, ctx->mt_alloc, ctx->part, T, ctx->ncu);
    launch_resid_w(st, x, ctx->part, gemm_planes(L.down, T, ctx->ncu), T, Mpad, H, round, next_ln1, next_ln1 ? ceil_div(H, 64) : 0,
                   next_ln1 ? ctx->xp_h : nullptr, ctx->ssp);
}

static int mpad_of(int T) { return 16 * ceil_div(T, 16) + (ceil_div(T, 16) > 1 && (ceil_div(T, 16) & 1) ? 16 : 0); }

// The blocks [p0, p1) (model indices) over the packed rows: blockSegs
// (web/model/model.js:619-624) per layer, with the reference's dispatches
// fused into: operand prep, q|k|v GEMM, finish (rmsnorm's row factor + RoPE +
// KV store + Q operand), attention, combine (o_proj operand), o GEMM,
// residual (+ operand x*ln2 and the row's sum of squares), gate|up GEMM,
// finish (row factor + SwiGLU), down GEMM, residual (+ round_f16 + the next
// block's operand x*ln1 and sum of squares). A linear_attention block
// replaces the attention half with linearBlockSegs (model.js:472-527).
static void run_blocks(cc_ctx* ctx, const StepPlan& p, const MetaLayout& ml, int b0, int b1) {
    const cc_dims& d = ctx->d;
    hipStream_t st = ctx->stream;
    const int T = p.T, H = d.hidden;
    const int Mpad = mpad_of(T);
    PassMeta pm;
    pm.jobs = (const JobDev*)(ctx->d_meta + ml.jobs);
    pm.items = (const AttnItem*)(ctx->d_meta + ml.items);
    pm.row_job = (const int32_t*)(ctx->d_meta + ml.row_job);
    pm.cwg = (const int32_t*)(ctx->d_meta + ml.cwg);
    pm.njobs = (int)p.jobs.size();
    pm.nitems = p.nitems;
    pm.nlaunch = p.nlaunch;
    pm.multi = p.multi;
    pm.ncwg = p.ncwg;
    const RowScale rs = row_scale_of(ctx);
    const int KUH = ceil_div(H, 64);   // every block's first matmul reads K = hidden
    int longest = 0;                   // a long job takes the row-parallel conv
    for (const JobDev& jd : p.jobs) longest = std::max(longest, (int)jd.n);
    for (int b = b0; b < b1; b++) {
        Layer& L = ctx->layers[b - ctx->L0];
        if (b == b0) launch_resid_w(st, ctx->x, nullptr, 0, T, Mpad, H, 0, L.ln1, KUH, ctx->xp_h, ctx->ssp);
        if (L.kind == CC_LINEAR_ATTENTION) {
            // linearBlockSegs (model.js:472-527): in_proj, conv + ring, the
            // recurrence on each session's state, gated norm, out_proj
            const LinGeom& lg = ctx->lg;
            launch_gemm(st, L.lin, ctx->xp_h, ctx->mt_alloc, ctx->part, T, ctx->ncu);
            if (longest > LIN_SEQ_ROWS)
                launch_lin_conv_rows(st, ctx->part, gemm_planes(L.lin, T, ctx->ncu), T, pm.njobs, pm.row_job, pm.jobs, rs, L.conv, lg, L.state,
                                     ctx->lraw, ctx->lrep, ctx->lring);
            else
                launch_lin_conv(st, ctx->part, gemm_planes(L.lin, T, ctx->ncu), T, pm.njobs, pm.jobs, rs, L.conv, lg, L.state, ctx->lraw,
                                ctx->lrep);
            launch_gdn(st, ctx->lraw, ctx->lrep, pm.njobs, pm.jobs, L.gp, lg, L.state, ctx->lcore);
            launch_lin_norm(st, ctx->lcore, ctx->lraw, L.gnorm, d.rms_eps, T, lg, L.out.KU, ctx->xp_v);
            launch_gemm(st, L.out, ctx->xp_v, ctx->mt_alloc, ctx->part, T, ctx->ncu);
            launch_resid_w(st, ctx->x, ctx->part, gemm_planes(L.out, T, ctx->ncu), T, Mpad, H, 0, L.ln2, KUH, ctx->xp_h, ctx->ssp);
        } else {
            full_attn_half(ctx, L, ctx->x, T, Mpad, pm);
        }
        const bool next = b + 1 < b1;
        ffn_half(ctx, L, ctx->x, T, Mpad, 1, next ? ctx->layers[b + 1 - ctx->L0].ln1 : nullptr);
    }
}

// mtpBlock's input (model.js:543-553): x = fc_e . enorm(embed_draft[ids]) +
// fc_h . hnorm(h), into ctx->mx, followed by the block's operand x*ln1 and
// its sums of squares. `ids` device int32 [T], `hin` rows [T][H]. The draft
// embedding is not rounded (gatherEmbedNoPos).
static void mtp_input(cc_ctx* ctx, const int32_t* ids, float* hin, int T) {
    const cc_dims& d = ctx->d;
    hipStream_t st = ctx->stream;
    const int H = d.hidden, KUH = ceil_div(H, 64), Mpad = mpad_of(T);
    launch_embed(st, ids, nullptr, T, ctx->embed_draft, ctx->mtp_e, 0);
    launch_resid_norm(st, ctx->mtp_e, nullptr, nullptr, 0, T, Mpad, H, 0, ctx->enorm, d.rms_eps, KUH, ctx->xp_e,
                      nullptr);
    launch_resid_norm(st, hin, nullptr, nullptr, 0, T, Mpad, H, 0, ctx->hnorm, d.rms_eps, KUH, ctx->xp_hh, nullptr);
    launch_gemm(st, ctx->fc_e, ctx->xp_e, ctx->mt_alloc, ctx->part, T, ctx->ncu);
    launch_sum_splits(st, ctx->part, gemm_planes(ctx->fc_e, T, ctx->ncu), T, H, ctx->mx);
    launch_gemm(st, ctx->fc_h, ctx->xp_hh, ctx->mt_alloc, ctx->part, T, ctx->ncu);
    launch_resid_w(st, ctx->mx, ctx->part, gemm_planes(ctx->fc_h, T, ctx->ncu), T, Mpad, H, 0, ctx->mtpL.ln1, KUH, ctx->xp_h, ctx->ssp);
}

// The MTP layer's KV rows for a pass's MTP jobs (stage.js:1404-1421): each
// row's token with the trunk's hidden row one position earlier (the
// session's kept row for row 0). Only K and V are wanted, so the block runs
// as far as the KV store: its output is not used (mtpBlock's is discarded).
static void mtp_fill(cc_ctx* ctx, const MetaLayout& ml, int Tm, int njobs) {
    hipStream_t st = ctx->stream;
    const cc_dims& d = ctx->d;
    const JobDev* mj = (const JobDev*)(ctx->d_meta + ml.mtp_jobs);
    const int32_t* mrow = (const int32_t*)(ctx->d_meta + ml.mtp_row_job);
    launch_gather_rows(st, ctx->x, ctx->mtpH, (const int32_t*)(ctx->d_meta + ml.mtp_src), Tm, d.hidden, ctx->mtp_in);
    mtp_input(ctx, (const int32_t*)(ctx->d_meta + ml.mtp_ids), ctx->mtp_in, Tm);
    Layer& M = ctx->mtpL;
    launch_gemm(st, M.qkv, ctx->xp_h, ctx->mt_alloc, ctx->part, Tm, ctx->ncu);
    QkExtras ex;
    if (ctx->hybrid) {   // k_norm applies; the gate's columns are in the planes but not read
        ex.qn = M.qn;
        ex.kn = M.kn;
        ex.eps = d.rms_eps;
        ex.gate = ctx->gbuf;
    }
    launch_fin_qkv(st, ctx->part, gemm_planes(M.qkv, Tm, ctx->ncu), Tm, mrow, mj, d.n_heads, ctx->group, ctx->geom, ctx->tbl, ctx->rot, M.kpool,
                   M.vpool, ctx->page_table, ctx->qp, row_scale_of(ctx), 0, 1, ex);
    (void)njobs;
}

// Profile replay (cc_profile): after the step's own work, each class's
// launches of that step run again back-to-back between one event pair, with
// every block's own weights and pools and the step's shapes. Launches queued
// back-to-back on one stream start as the previous one ends, so the pair's
// interval over n launches is n kernel durations with no marker between them
// (a marker next to every launch costs each a few microseconds of gap). The
// replays write only scratch the step has consumed (matmul planes, attention
// partials) or, for the head, the same logits again from the same operand.
static void prof_replay(cc_ctx* ctx, const StepPlan& p, const MetaLayout& ml, int b0, int b1, bool head) {
    const cc_dims& d = ctx->d;
    hipStream_t st = ctx->stream;
    const int T = p.T;
    const JobDev* djobs = (const JobDev*)(ctx->d_meta + ml.jobs);
    const AttnItem* ditems = (const AttnItem*)(ctx->d_meta + ml.items);
    // (a linear_attention block has no q|k|v, o or KV: its matmuls are not replayed)
    auto blocks = [&](int kind, QTensor Layer::*w, const uint4* xp) {
        double bytes = 0;
        int n = 0;
        for (int b = b0; b < b1; b++)
            if ((ctx->layers[b - ctx->L0].*w).codes) {
                bytes += qbytes(ctx->layers[b - ctx->L0].*w);
                n++;
            }
        if (n == 0) return;
        prof_mark(ctx, kind, n, bytes, [&] {
            for (int b = b0; b < b1; b++)
                if ((ctx->layers[b - ctx->L0].*w).codes)
                    launch_gemm(st, ctx->layers[b - ctx->L0].*w, xp, ctx->mt_alloc, ctx->part, T, ctx->ncu);
        });
    };
    if (b1 > b0) {
        blocks(CC_K_QKV, &Layer::qkv, ctx->xp_h);
        int nfull = 0;
        for (int b = b0; b < b1; b++) nfull += ctx->layers[b - ctx->L0].kpool != nullptr;
        if (p.nitems > 0 && nfull > 0)
            prof_mark(ctx, CC_K_ATTN, nfull, p.kv_bytes * nfull, [&] {
                for (int b = b0; b < b1; b++) {
                    const Layer& L = ctx->layers[b - ctx->L0];
                    if (!L.kpool) continue;
                    launch_attn(st, ditems, p.nlaunch, ctx->qp, L.kpool, L.vpool, ctx->page_table, ctx->geom,
                                ctx->group, ctx->ppw, ctx->apart, p.multi, ctx->attn);
                }
            });
        blocks(CC_K_O, &Layer::o, ctx->xp_o);
        blocks(CC_K_GU, &Layer::gu, ctx->xp_h);
        blocks(CC_K_DOWN, &Layer::down, ctx->xp_f);
    }
    if (head) {
        const QTensor& hw = d.tied ? ctx->wte : ctx->lm_head;
        prof_mark(ctx, CC_K_HEAD, 1, qbytes(hw), [&] { launch_gemm(st, hw, ctx->xp_h, ctx->mt_alloc, ctx->logits, p.S, ctx->ncu); });
    }
}

// k_pack over the PackJobs the pass uploaded, each past advanced by `step`.
static void pack_on_device(cc_ctx* ctx, const MetaLayout& ml, int njobs, int step, bool head) {
    PackGeom g{ctx->geom.nKV, ctx->group, ctx->geom.ng, ctx->D, ctx->ppw, ctx->geom.page, head ? 1 : 0};
    uint8_t* dm = ctx->d_meta;
    launch_pack(ctx->stream, (const PackJob*)(dm + ml.pack), njobs, step, g, (JobDev*)(dm + ml.jobs),
                (AttnItem*)(dm + ml.items), (int32_t*)(dm + ml.row_job), (int32_t*)(dm + ml.head_rows),
                (int32_t*)(dm + ml.cwg));
}

cc_status cc_step(cc_ctx* ctx, const cc_job* jobs, int32_t njobs, int32_t at, int32_t to, int32_t topk,
                  float* top_vals, uint32_t* top_ids, uint16_t* hidden_out, int32_t* status) {
    if (!ctx) return CC_EARG;
    const cc_dims& d = ctx->d;
    const int positions = d.n_layer + 2;
    if (status) for (int j = 0; j < njobs; j++) status[j] = CC_OK;
    auto bad = [&](int j, const std::string& msg) {
        if (status && j >= 0) status[j] = CC_EARG;
        return fail(ctx, CC_EARG, msg);
    };
    if (!jobs || njobs < 1 || njobs > ctx->o.max_jobs) return bad(-1, "1..max_jobs jobs per pass");
    if (at < ctx->o.lo || at >= ctx->o.hi || to <= at || to > ctx->o.hi)
        return bad(-1, "positions " + std::to_string(at) + ".." + std::to_string(to) + " are not held here");
    const bool gather = at == 0;
    // A pass to the end of the line samples its jobs' `sampled` rows; with
    // none (a prefill chunk's fill or a replay, web/model/stage.js:1219-1222)
    // it only writes the caches and runs no LM head.
    const bool at_end = to == positions;
    int S_all = 0;
    for (int j = 0; j < njobs && jobs; j++) S_all += at_end ? std::max(0, jobs[j].sampled) : 0;
    const bool head = at_end && S_all > 0;
    if (head && (topk < 1 || topk > TOPK_MAX)) return bad(-1, "topk must be 1..256");
    if (head && (!top_vals || !top_ids)) return bad(-1, "a pass to the head needs top_vals and top_ids");
    if (!at_end && !hidden_out) return bad(-1, "a pass that stops before the head needs hidden_out");
    int T = 0;
    std::vector<char> seen(ctx->owned.size(), 0);
    // #prepare's checks (web/model/stage.js:1225-1259).
    for (int j = 0; j < njobs; j++) {
        const cc_job& jb = jobs[j];
        if (jb.slot < 0 || jb.slot >= (int)ctx->owned.size()) return bad(j, "slot out of range");
        if (seen[jb.slot]) return bad(j, "one job per session in a pass");
        seen[jb.slot] = 1;
        if (jb.n < 1 || jb.n > ctx->o.t_max)
            return bad(j, "a job of " + std::to_string(jb.n) + " tokens is outside 1-" + std::to_string(ctx->o.t_max));
        if (jb.past < 0) return bad(j, "past " + std::to_string(jb.past) + " is not a position");
        if (jb.past + jb.n > ctx->o.n_max)
            return bad(j, "context " + std::to_string(jb.past + jb.n) + " exceeds " + std::to_string(ctx->o.n_max));
        if (gather) {
            if (!jb.ids) return bad(j, "a job at position 0 needs " + std::to_string(jb.n) + " token ids");
            for (int i = 0; i < jb.n; i++)
                if (jb.ids[i] < 0 || jb.ids[i] >= d.vocab) return bad(j, "a token id is outside the vocabulary");
        } else if (!jb.hidden) {
            return bad(j, "a job past position 0 needs its hidden rows");
        }
        if (at_end && !(jb.sampled == 0 || jb.sampled == 1 || jb.sampled == jb.n))
            return bad(j, "sampled must be 0, 1 or n at the head");
        if (jb.mtp && ctx->mtp && at_end) {
            // the MTP fill pairs each row's token with the row before (stage.js:1293)
            if (!jb.ids) return bad(j, "an MTP job needs its " + std::to_string(jb.n) + " token ids");
            for (int i = 0; i < jb.n; i++)
                if (jb.ids[i] < 0 || jb.ids[i] >= d.vocab) return bad(j, "a token id is outside the vocabulary");
        }
        if (ctx->any_linear) {
            // A recurrent block cannot be rewound, only restarted (past 0) or
            // rolled back to before its last verify (stage.js:1028-1090).
            if (jb.snap && jb.n > LIN_SPEC_ROWS)
                return bad(j, "a verify job has at most " + std::to_string(LIN_SPEC_ROWS) + " rows");
            const int sb = ctx->spec_base[jb.slot], sn = ctx->spec_n[jb.slot];
            if (jb.rollback && (sn < 0 || jb.keep < 0 || jb.keep > sn || jb.past != sb + jb.keep)) {
                if (status) status[j] = CC_COLD;
                return fail(ctx, CC_COLD, "session " + std::to_string(jb.slot) +
                                              " has no replay data here to roll back to " + std::to_string(jb.past));
            }
            if (!jb.rollback && jb.past > 0 && jb.past != ctx->fed[jb.slot]) {
                if (status) status[j] = CC_COLD;
                return fail(ctx, CC_COLD, "session " + std::to_string(jb.slot) + " is no longer cached here (its " +
                                              "recurrent blocks hold " + std::to_string(ctx->fed[jb.slot]) +
                                              " rows, the job continues from " + std::to_string(jb.past) + ")");
            }
        }
        T += jb.n;
    }
    if (T > ctx->o.t_max) return bad(-1, "the pass has " + std::to_string(T) + " rows, above t_max");

    StepPlan p;
    plan_jobs(ctx, jobs, njobs, p, head);
    if (std::max(p.nitems, p.nlaunch) > (int)ctx->items_cap || (size_t)p.ncwg > max_cwg_for(ctx))
        return bad(-1, "too many attention items");
    cc_status gs = grow(ctx, p);
    if (gs != CC_OK) return gs;
    MetaLayout ml = meta_layout(ctx);
    uint8_t* hm = ctx->h_meta;
    // the jobs for the device packer (k_pack builds the pass's tables)
    PackJob* pk = (PackJob*)(hm + ml.pack);
    for (int j = 0; j < njobs; j++)
        pk[j] = PackJob{jobs[j].slot, jobs[j].past, jobs[j].n, head ? jobs[j].sampled : 0, p.jobs[j].snap,
                        p.jobs[j].keep};
    std::vector<std::pair<int, int>> want;
    for (int j = 0; j < njobs; j++) want.push_back({jobs[j].slot, jobs[j].past + jobs[j].n});
    {
        // Page plan (host counts), written before the copy.
        int32_t* plan = (int32_t*)(hm + ml.plan);
        int total = 0;
        for (int j = 0; j < njobs; j++) {
            const int need = ceil_div(want[j].second, ctx->geom.page);
            const int nw = std::max(0, need - ctx->owned[want[j].first]);
            plan[4 * j] = want[j].first;
            plan[4 * j + 1] = ctx->owned[want[j].first];
            plan[4 * j + 2] = nw;
            plan[4 * j + 3] = total;
            total += nw;
        }
    }
    size_t copy_bytes = ml.hidden;
    // The MTP jobs' rows, packed (stage.js:1404-1421): row 0 of a job pairs
    // its first token with the session's kept row, row i with the job's row
    // i - 1.
    int Tm = 0, nmj = 0;
    if (ctx->mtp && at_end) {
        JobDev* mj = (JobDev*)(hm + ml.mtp_jobs);
        int32_t* mrow = (int32_t*)(hm + ml.mtp_row_job);
        int32_t* msrc = (int32_t*)(hm + ml.mtp_src);
        int32_t* mids = (int32_t*)(hm + ml.mtp_ids);
        for (int j = 0; j < njobs; j++) {
            if (!jobs[j].mtp) continue;
            JobDev jd = p.jobs[j];
            jd.row0 = Tm;
            jd.qp_off = 0;
            jd.snap = 0;
            jd.keep = -1;
            for (int i = 0; i < jobs[j].n; i++) {
                mrow[Tm + i] = nmj;
                msrc[Tm + i] = i == 0 ? -1 - jobs[j].slot : p.jobs[j].row0 + i - 1;
                mids[Tm + i] = jobs[j].ids[i];
            }
            mj[nmj++] = jd;
            Tm += jobs[j].n;
        }
    }
    if (gather) {
        int32_t* ids = (int32_t*)(hm + ml.ids);
        int r = 0;
        for (int j = 0; j < njobs; j++)
            for (int i = 0; i < jobs[j].n; i++) ids[r++] = jobs[j].ids[i];
    } else {
        uint16_t* hid = (uint16_t*)(hm + ml.hidden);
        size_t r = 0;
        for (int j = 0; j < njobs; j++) {
            std::memcpy(hid + r, jobs[j].hidden, (size_t)jobs[j].n * d.hidden * 2);
            r += (size_t)jobs[j].n * d.hidden;
        }
        copy_bytes = ml.hidden + (size_t)T * d.hidden * 2;
    }
    hipStream_t st = ctx->stream;
    HIPCHK(hipEventRecord(ctx->ev0, st));
    HIPCHK(hipMemcpyAsync(ctx->d_meta, hm, copy_bytes, hipMemcpyHostToDevice, st));
    pack_on_device(ctx, ml, njobs, 0, head);
    cc_status ps = take_pages(ctx, want, (int32_t*)(ctx->d_meta + ml.plan), (int32_t*)(hm + ml.plan), status);
    if (ps != CC_OK) {
        (void)hipStreamSynchronize(st);   // the refusal is the status reported
        return ps;
    }
    // Embedding (position 0) or the rows handed in.
    QTensor emb = ctx->wte;
    emb.K = d.hidden;
    if (gather) launch_embed(st, (const int32_t*)(ctx->d_meta + ml.ids), nullptr, T, emb, ctx->x);
    else {
        QTensor shape;
        shape.K = d.hidden;
        launch_embed(st, nullptr, (const uint16_t*)(ctx->d_meta + ml.hidden), T, shape, ctx->x);
    }
    const int b0 = std::max(at, 1) - 1, b1 = std::min(to, d.n_layer + 1) - 1;
    if (b1 > b0) run_blocks(ctx, p, ml, b0, b1);
    void* hout = ctx->h_out;
    if (head) {
        const QTensor& hw = d.tied ? ctx->wte : ctx->lm_head;
        const int S = p.S;
        const int Mpad = 32 * ceil_div(S, 32);
        launch_resid_norm(st, ctx->x, (const int32_t*)(ctx->d_meta + ml.head_rows), nullptr, 0, S, Mpad, d.hidden, 0,
                          ctx->norm, d.rms_eps, hw.KU, ctx->xp_h, nullptr);
        launch_gemm(st, hw, ctx->xp_h, ctx->mt_alloc, ctx->logits, S, ctx->ncu);
        ctx->head_rows = S;
        launch_topk(st, ctx->logits, gemm_planes(hw, S, ctx->ncu), S, d.vocab, topk, ctx->tk_a, ctx->tk_b, ctx->d_vals, ctx->d_ids);
        HIPCHK(hipMemcpyAsync(hout, ctx->d_vals, (size_t)S * topk * 4, hipMemcpyDeviceToHost, st));
        HIPCHK(hipMemcpyAsync((uint8_t*)hout + (size_t)S * topk * 4, ctx->d_ids, (size_t)S * topk * 4,
                              hipMemcpyDeviceToHost, st));
    } else if (!at_end) {
        launch_to_half_bits(st, ctx->x, (int64_t)T * d.hidden, ctx->d_hbits);
        HIPCHK(hipMemcpyAsync(hout, ctx->d_hbits, (size_t)T * d.hidden * 2, hipMemcpyDeviceToHost, st));
    }
    if (Tm > 0) {
        mtp_fill(ctx, ml, Tm, nmj);
        // a job that samples nothing (a prefill chunk) keeps its last row for
        // the next job's row 0; a sampled job's row is kept by cc_mtp_draft
        for (int j = 0; j < njobs; j++)
            if (jobs[j].mtp && jobs[j].sampled == 0)
                HIPCHK(hipMemcpyAsync(ctx->mtpH + (size_t)jobs[j].slot * d.hidden,
                                      ctx->x + (size_t)(p.jobs[j].row0 + jobs[j].n - 1) * d.hidden,
                                      (size_t)d.hidden * 4, hipMemcpyDeviceToDevice, st));
    }
    HIPCHK(hipEventRecord(ctx->ev1, st));
    if (ctx->prof) prof_replay(ctx, p, ml, b0, b1, head);
    HIPCHK(hipStreamSynchronize(st));
    HIPCHK(take_launch_error());
    float ms = 0;
    if (hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1) != hipSuccess) ms = 0;
    ctx->last_ms = ms;
    prof_collect(ctx);
    ctx->passes++;
    ctx->rows += T;
    ctx->last_T = T;
    if (b1 > b0) {
        // what the recurrent blocks now hold, and the verify a rollback may return to
        for (int j = 0; j < njobs; j++) {
            const int sl = jobs[j].slot;
            ctx->fed[sl] = jobs[j].past + jobs[j].n;
            if (jobs[j].snap) {
                ctx->spec_base[sl] = jobs[j].past;
                ctx->spec_n[sl] = jobs[j].n;
            } else {
                ctx->spec_n[sl] = -1;
            }
        }
    }
    if (head) {
        std::memcpy(top_vals, hout, (size_t)p.S * topk * 4);
        std::memcpy(top_ids, (uint8_t*)hout + (size_t)p.S * topk * 4, (size_t)p.S * topk * 4);
    } else if (!at_end) {
        std::memcpy(hidden_out, hout, (size_t)T * d.hidden * 2);
    }
    return CC_OK;
}

cc_status cc_decode_steps(cc_ctx* ctx, const cc_job* jobs, int32_t njobs, int32_t steps, int32_t topk,
                          float* top_vals, uint32_t* top_ids) {
    if (!ctx) return CC_EARG;
    const cc_dims& d = ctx->d;
    const int positions = d.n_layer + 2;
    if (ctx->o.lo != 0 || ctx->o.hi != positions)
        return fail(ctx, CC_EARG, "a decode loop needs every position (0.." + std::to_string(positions - 1) + ") here");
    if (ctx->any_linear || ctx->mtp)
        return fail(ctx, CC_EARG, "a decode loop runs full-attention models without an MTP head");
    if (!jobs || njobs < 1 || njobs > ctx->o.max_jobs) return fail(ctx, CC_EARG, "1..max_jobs jobs per pass");
    if (steps < 1) return fail(ctx, CC_EARG, "steps must be positive");
    if (topk < 1 || topk > TOPK_MAX) return fail(ctx, CC_EARG, "topk must be 1..256");
    if (!top_vals || !top_ids) return fail(ctx, CC_EARG, "a decode loop needs top_vals and top_ids");
    if (njobs > ctx->o.t_max) return fail(ctx, CC_EARG, "the pass has more rows than t_max");
    std::vector<char> seen(ctx->owned.size(), 0);
    for (int j = 0; j < njobs; j++) {
        const cc_job& jb = jobs[j];
        if (jb.slot < 0 || jb.slot >= (int)ctx->owned.size()) return fail(ctx, CC_EARG, "slot out of range");
        if (seen[jb.slot]) return fail(ctx, CC_EARG, "one job per session in a pass");
        seen[jb.slot] = 1;
        if (jb.n != 1 || jb.sampled != 1 || jb.snap || jb.rollback || jb.mtp)
            return fail(ctx, CC_EARG, "a decode loop takes one-row jobs, each sampled");
        if (!jb.ids || jb.ids[0] < 0 || jb.ids[0] >= d.vocab)
            return fail(ctx, CC_EARG, "a job at position 0 needs 1 token ids");
        if (jb.past < 0 || jb.past + steps > ctx->o.n_max)
            return fail(ctx, CC_EARG, "context " + std::to_string(jb.past + steps) + " exceeds " +
                                          std::to_string(ctx->o.n_max));
    }
    // plans of the first and the last step: the last needs the most items
    std::vector<cc_job> last(jobs, jobs + njobs);
    for (auto& j : last) j.past += steps - 1;
    StepPlan pl;
    plan_jobs(ctx, last.data(), njobs, pl, true);
    if (std::max(pl.nitems, pl.nlaunch) > (int)ctx->items_cap || (size_t)pl.ncwg > max_cwg_for(ctx))
        return fail(ctx, CC_EARG, "too many attention items");
    cc_status gs = grow(ctx, pl);
    if (gs != CC_OK) return gs;
    const int S = njobs;
    const size_t per = (size_t)S * topk;
    if (per * steps > ctx->dec_cap) {
        float* v = nullptr;
        uint32_t* i = nullptr;
        HIPCHK(dfree(ctx, ctx->dec_vals, ctx->dec_cap * 4, &ctx->scratch_bytes));
        HIPCHK(dfree(ctx, ctx->dec_ids, ctx->dec_cap * 4, &ctx->scratch_bytes));
        ctx->dec_vals = nullptr;
        ctx->dec_ids = nullptr;
        ctx->dec_cap = 0;
        HIPCHK(dalloc(ctx, &v, per * steps * 4, &ctx->scratch_bytes));
        HIPCHK(dalloc(ctx, &i, per * steps * 4, &ctx->scratch_bytes));
        ctx->dec_vals = v;
        ctx->dec_ids = i;
        ctx->dec_cap = per * steps;
    }
    // Pages as a host loop of cc_step calls takes them (take_pages, after
    // ensurePages, web/model/model.js:185-202): pass k pops, job by job in
    // order, the pages its past + k + 1 tokens need beyond those it owns.
    // Every pass's pops are planned here, (slot, owned, new pages, prefix in
    // the pass) for each job that takes one, and an allocating pass runs its
    // plan first, so the frames end with the page tables the Runner's passes
    // give them.
    std::vector<int32_t> pplan;
    std::vector<int> pass_off(steps + 1, 0), pass_top(steps, 0);
    std::vector<int> own(ctx->owned);
    int top = ctx->top;
    for (int k = 0; k < steps; k++) {
        pass_off[k] = (int)(pplan.size() / 4);
        pass_top[k] = top;
        int pre = 0;
        for (int j = 0; j < njobs; j++) {
            const int slot = jobs[j].slot;
            const int nw = ceil_div(jobs[j].past + k + 1, ctx->geom.page) - own[slot];
            if (nw <= 0) continue;
            pplan.insert(pplan.end(), {slot, own[slot], nw, pre});
            pre += nw;
            own[slot] += nw;
        }
        if (pre > top)
            return fail(ctx, CC_BUSY, "no KV page free for pass " + std::to_string(k) + " of the loop (" +
                                          std::to_string(pre) + " needed, " + std::to_string(top) + " free)");
        top -= pre;
    }
    pass_off[steps] = (int)(pplan.size() / 4);
    if (pplan.size() > ctx->dec_plan_cap) {
        int32_t* dp = nullptr;
        HIPCHK(dfree(ctx, ctx->dec_plan, ctx->dec_plan_cap * 4, &ctx->scratch_bytes));
        ctx->dec_plan = nullptr;
        ctx->dec_plan_cap = 0;
        HIPCHK(dalloc(ctx, &dp, pplan.size() * 4, &ctx->scratch_bytes));
        ctx->dec_plan = dp;
        ctx->dec_plan_cap = pplan.size();
    }
    MetaLayout ml = meta_layout(ctx);
    uint8_t* hm = ctx->h_meta;
    PackJob* pk = (PackJob*)(hm + ml.pack);
    int32_t* ids0 = (int32_t*)(hm + ml.ids);
    for (int j = 0; j < njobs; j++) {
        pk[j] = PackJob{jobs[j].slot, jobs[j].past, 1, 1, 0, -1};
        ids0[j] = jobs[j].ids[0];
    }
    hipStream_t st = ctx->stream;
    HIPCHK(hipEventRecord(ctx->ev0, st));
    HIPCHK(hipMemcpyAsync(ctx->d_meta, hm, ml.hidden, hipMemcpyHostToDevice, st));
    if (!pplan.empty())
        HIPCHK(hipMemcpyAsync(ctx->dec_plan, pplan.data(), pplan.size() * 4, hipMemcpyHostToDevice, st));
    const QTensor& hw = d.tied ? ctx->wte : ctx->lm_head;
    QTensor emb = ctx->wte;
    emb.K = d.hidden;
    int32_t* d_ids_in = (int32_t*)(ctx->d_meta + ml.ids);
    const int Mpad = 32 * ceil_div(S, 32);
    std::vector<cc_job> cur(jobs, jobs + njobs);
    for (int k = 0; k < steps; k++) {
        // step k: every job one row further, fed the token step k-1 sampled
        launch_alloc_pages(st, ctx->dec_plan + 4 * (size_t)pass_off[k], pass_off[k + 1] - pass_off[k],
                           ctx->free_stack, pass_top[k], ctx->page_table, ctx->max_pages);
        StepPlan p;
        plan_jobs(ctx, cur.data(), njobs, p, true);
        pack_on_device(ctx, ml, njobs, k, true);
        if (k > 0) launch_ids_col0(st, ctx->dec_ids + (k - 1) * per, S, topk, d_ids_in);
        launch_embed(st, d_ids_in, nullptr, p.T, emb, ctx->x);
        run_blocks(ctx, p, ml, 0, d.n_layer);
        launch_resid_norm(st, ctx->x, (const int32_t*)(ctx->d_meta + ml.head_rows), nullptr, 0, S, Mpad, d.hidden, 0,
                          ctx->norm, d.rms_eps, hw.KU, ctx->xp_h, nullptr);
        launch_gemm(st, hw, ctx->xp_h, ctx->mt_alloc, ctx->logits, S, ctx->ncu);
        launch_topk(st, ctx->logits, gemm_planes(hw, S, ctx->ncu), S, d.vocab, topk, ctx->tk_a, ctx->tk_b, ctx->dec_vals + k * per,
                    ctx->dec_ids + k * per);
        for (auto& j : cur) j.past++;
    }
    ctx->head_rows = S;
    ctx->owned = own;
    ctx->top = top;
    HIPCHK(hipMemcpyAsync(top_vals, ctx->dec_vals, per * steps * 4, hipMemcpyDeviceToHost, st));
    HIPCHK(hipMemcpyAsync(top_ids, ctx->dec_ids, per * steps * 4, hipMemcpyDeviceToHost, st));
    HIPCHK(hipEventRecord(ctx->ev1, st));
    HIPCHK(hipStreamSynchronize(st));
    HIPCHK(take_launch_error());
    float ms = 0;
    if (hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1) != hipSuccess) ms = 0;
    ctx->last_ms = ms;
    ctx->passes += steps;
    ctx->rows += (int64_t)steps * njobs;
    ctx->last_T = njobs;
    for (int j = 0; j < njobs; j++) {
        ctx->fed[jobs[j].slot] = jobs[j].past + steps;
        ctx->spec_n[jobs[j].slot] = -1;
    }
    return CC_OK;
}

cc_status cc_mtp_draft(cc_ctx* ctx, int32_t slot, int32_t row, int32_t token, int32_t pos, int32_t k_drafts,
                       uint32_t* drafts) {
    if (!ctx) return CC_EARG;
    if (!ctx->mtp) return fail(ctx, CC_EARG, "no MTP head here");
    const cc_dims& d = ctx->d;
    const int H = d.hidden, K = k_drafts;
    if (slot < 0 || slot >= (int)ctx->owned.size()) return fail(ctx, CC_EARG, "bad slot");
    if (row < -1 || row >= ctx->last_T) return fail(ctx, CC_EARG, "row is not a row of the last pass");
    if (K < 0 || K > MTP_STEPS_MAX) return fail(ctx, CC_EARG, "0..7 drafts");
    if (K > 0 && (token < 0 || token >= d.mtp_vocab)) return fail(ctx, CC_EARG, "the token is outside the draft rows");
    if (K > 0 && (pos < 0 || pos + K > ctx->o.n_max)) return fail(ctx, CC_EARG, "the drafts pass the context window");
    if (K > 0 && !drafts) return fail(ctx, CC_EARG, "null drafts");
    hipStream_t st = ctx->stream;
    float* kept = ctx->mtpH + (size_t)slot * H;
    if (row >= 0) HIPCHK(hipMemcpyAsync(kept, ctx->x + (size_t)row * H, (size_t)H * 4, hipMemcpyDeviceToDevice, st));
    if (K == 0) {
        HIPCHK(hipStreamSynchronize(st));
        return CC_OK;
    }
    // pages for the draft rows (stage.js:1291: the head takes them with the job)
    {
        int32_t* h_plan = (int32_t*)ctx->h_meta;
        int32_t* d_plan = (int32_t*)ctx->d_meta;
        HIPCHK(hipStreamSynchronize(st));
        const int need = ceil_div(pos + K, ctx->geom.page);
        h_plan[0] = slot;
        h_plan[1] = ctx->owned[slot];
        h_plan[2] = std::max(0, need - ctx->owned[slot]);
        h_plan[3] = 0;
        HIPCHK(hipMemcpyAsync(d_plan, h_plan, 16, hipMemcpyHostToDevice, st));
        std::vector<std::pair<int, int>> want{{slot, pos + K}};
        cc_status ps = take_pages(ctx, want, d_plan, h_plan, nullptr);
        if (ps != CC_OK) return ps;
    }
    // every step's one-row plan, in one upload; ids[0] the token, ids[k+1]
    // step k's draft (written on the device, read by step k+1)
    std::vector<StepPlan> plans(K);
    uint8_t* hc = ctx->h_chain;
    ((int32_t*)hc)[0] = token;
    const size_t mtq1 = ceil_div(ctx->group, 16);
    const size_t a256 = 255;
    auto al = [&](size_t b) { return (b + a256) & ~a256; };
    const size_t o_items = al(sizeof(JobDev)), o_row = o_items + al(sizeof(AttnItem) * ctx->geom.nKV * mtq1 *
                                                                     ceil_div(ctx->max_pages, ctx->ppw));
    const size_t o_cwg = o_row + al(4);
    for (int k = 0; k < K; k++) {
        cc_job j{};
        j.slot = slot;
        j.past = pos + k;
        j.n = 1;
        build_plan(ctx, &j, 1, plans[k], false);
        uint8_t* b = hc + 256 + (size_t)k * ctx->chain_step;
        if (o_items + plans[k].items.size() * sizeof(AttnItem) > o_row || plans[k].cwg.size() * 4 > 12 * ctx->geom.nKV * mtq1)
            return fail(ctx, CC_EARG, "draft step plan too large");
        std::memcpy(b, plans[k].jobs.data(), sizeof(JobDev));
        std::memcpy(b + o_items, plans[k].items.data(), plans[k].items.size() * sizeof(AttnItem));
        std::memcpy(b + o_row, plans[k].row_job.data(), 4);
        std::memcpy(b + o_cwg, plans[k].cwg.data(), plans[k].cwg.size() * 4);
    }
    HIPCHK(hipMemcpyAsync(ctx->d_chain, hc, 256 + (size_t)K * ctx->chain_step, hipMemcpyHostToDevice, st));
    int32_t* ids = (int32_t*)ctx->d_chain;
    HIPCHK(hipMemcpyAsync(ctx->mtp_in, kept, (size_t)H * 4, hipMemcpyDeviceToDevice, st));
    const int KUH = ceil_div(H, 64);
    for (int k = 0; k < K; k++) {
        // mtpChain step k (model.js:567-576): mtpBlock then mtpDraft
        const uint8_t* b = ctx->d_chain + 256 + (size_t)k * ctx->chain_step;
        PassMeta pm;
        pm.jobs = (const JobDev*)b;
        pm.items = (const AttnItem*)(b + o_items);
        pm.row_job = (const int32_t*)(b + o_row);
        pm.cwg = (const int32_t*)(b + o_cwg);
        pm.njobs = 1;
        pm.nitems = plans[k].nitems;
        pm.nlaunch = plans[k].nlaunch;
        pm.multi = plans[k].multi;
        pm.ncwg = plans[k].ncwg;
        mtp_input(ctx, ids + k, ctx->mtp_in, 1);
        full_attn_half(ctx, ctx->mtpL, ctx->mx, 1, mpad_of(1), pm);
        ffn_half(ctx, ctx->mtpL, ctx->mx, 1, mpad_of(1), 0, nullptr);
        launch_resid_norm(st, ctx->mx, nullptr, nullptr, 0, 1, 32, H, 0, ctx->mtp_norm, d.rms_eps, KUH, ctx->xp_h,
                          nullptr);
        launch_gemm(st, ctx->head_draft, ctx->xp_h, ctx->mt_alloc, ctx->mtp_logits, 1, ctx->ncu);
        launch_topk(st, ctx->mtp_logits, gemm_planes(ctx->head_draft, 1, ctx->ncu), 1, d.mtp_vocab, 1, ctx->tk_a, ctx->tk_b, ctx->d_vals,
                    (uint32_t*)(ids + k + 1));
        if (k + 1 < K)
            HIPCHK(hipMemcpyAsync(ctx->mtp_in, ctx->mx, (size_t)H * 4, hipMemcpyDeviceToDevice, st));
    }
    HIPCHK(hipMemcpyAsync(drafts, ids + 1, (size_t)K * 4, hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    HIPCHK(take_launch_error());
    return CC_OK;
}

// ------------------------------------------------------ kernel-level ops ---
cc_status cc_op_matmul_q8(cc_ctx* ctx, const float* X, int32_t M, int32_t K, const int8_t* W,
                          const uint16_t* scales_f16, int32_t N, float* Y) {
    if (!ctx || !X || !W || !scales_f16 || !Y || M < 1 || K < 4 || N < 1 || K % 4) return fail(ctx, CC_EARG, "bad matmul");
    QTensor q{};
    q.N = N;
    q.K = K;
    q.Nt = ceil_div(ceil_div(N, 16), 2) * 2;
    q.KU = ceil_div(K, 64);
    q.P = lx_planes_for(N, K, ctx->ncu);
    const int ng = ceil_div(K, 32);
    const int Mt = 2 * ceil_div(M, 32);
    const int sp = q.P;
    int8_t* dW = nullptr; uint16_t* dS = nullptr; float* dX = nullptr; float* dP = nullptr; float* dY = nullptr;
    uint4* dXp = nullptr;
    HIPCHK(hipMalloc(&q.codes, (size_t)q.Nt * q.KU * (LX_REC / 2)));
    HIPCHK(hipMemsetAsync(q.codes, 0, (size_t)q.Nt * q.KU * (LX_REC / 2), ctx->stream));
    HIPCHK(hipMalloc(&dW, (size_t)N * K));
    HIPCHK(hipMalloc(&dS, (size_t)N * ng * 2));
    HIPCHK(hipMalloc(&dX, (size_t)M * K * 4));
    HIPCHK(hipMalloc(&dXp, (size_t)Mt * 2 * q.KU * 2 * 1024));
    HIPCHK(hipMalloc(&dP, (size_t)sp * M * N * 4));
    HIPCHK(hipMalloc(&dY, (size_t)M * N * 4));
    HIPCHK(hipMemcpy(dW, W, (size_t)N * K, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(dS, scales_f16, (size_t)N * ng * 2, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(dX, X, (size_t)M * K * 4, hipMemcpyHostToDevice));
    hipStream_t st = ctx->stream;
    launch_tile_q8(st, dW, dS, N, K, q, 0);
    launch_prep_rows(st, dX, K, M, Mt * 16, K, q.KU, dXp);
    launch_gemm(st, q, dXp, Mt, dP, M, ctx->ncu);
    launch_sum_splits(st, dP, gemm_planes(q, M, ctx->ncu), M, N, dY);
    HIPCHK(hipStreamSynchronize(st));
    HIPCHK(take_launch_error());
    HIPCHK(hipMemcpy(Y, dY, (size_t)M * N * 4, hipMemcpyDeviceToHost));
    for (void* v : {(void*)q.codes, (void*)dW, (void*)dS, (void*)dX, (void*)dXp, (void*)dP, (void*)dY})
        (void)hipFree(v);
    return CC_OK;
}

cc_status cc_op_round_f16(cc_ctx* ctx, float* a, int64_t n) {
    if (!ctx || !a || n < 0) return CC_EARG;
    float* dA = nullptr;
    HIPCHK(hipMalloc(&dA, (size_t)n * 4 + 16));
    HIPCHK(hipMemcpy(dA, a, (size_t)n * 4, hipMemcpyHostToDevice));
    launch_round_f16(ctx->stream, dA, n);
    HIPCHK(hipStreamSynchronize(ctx->stream));
    HIPCHK(hipMemcpy(a, dA, (size_t)n * 4, hipMemcpyDeviceToHost));
    (void)hipFree(dA);
    return CC_OK;
}

cc_status cc_op_topk(cc_ctx* ctx, const float* logits, int32_t rows, int32_t V, int32_t M, float* vals,
                     uint32_t* ids) {
    if (!ctx || !logits || rows < 1 || V < 1 || M < 1 || M > TOPK_MAX || M > V) return fail(ctx, CC_EARG, "bad topk");
    float* dL = nullptr; uint64_t* a = nullptr; uint64_t* b = nullptr; float* dv = nullptr; uint32_t* di = nullptr;
    const size_t keys = (size_t)rows * ceil_div(V, 4096) * M + 16;
    HIPCHK(hipMalloc(&dL, (size_t)rows * V * 4));
    HIPCHK(hipMalloc(&a, keys * 8));
    HIPCHK(hipMalloc(&b, keys * 8));
    HIPCHK(hipMalloc(&dv, (size_t)rows * M * 4));
    HIPCHK(hipMalloc(&di, (size_t)rows * M * 4));
    HIPCHK(hipMemcpy(dL, logits, (size_t)rows * V * 4, hipMemcpyHostToDevice));
    launch_topk(ctx->stream, dL, 1, rows, V, M, a, b, dv, di);
    HIPCHK(hipStreamSynchronize(ctx->stream));
    HIPCHK(hipMemcpy(vals, dv, (size_t)rows * M * 4, hipMemcpyDeviceToHost));
    HIPCHK(hipMemcpy(ids, di, (size_t)rows * M * 4, hipMemcpyDeviceToHost));
    for (void* v : {(void*)dL, (void*)a, (void*)b, (void*)dv, (void*)di}) (void)hipFree(v);
    return CC_OK;
}

cc_status cc_topk_noalloc(cc_ctx* ctx, const float* logits, int32_t rows, int32_t V, int32_t M, float* vals,
                          uint32_t* ids, void* stream) {
    if (!ctx) return CC_EARG;
    if (!logits || !vals || !ids || rows < 1 || V < 1 || M < 1 || M > TOPK_MAX || M > V)
        return fail(ctx, CC_EARG, "bad topk: rows >= 1, 1 <= M <= min(V, 256), and device buffers");
    if (!ctx->tk_scratch) return fail(ctx, CC_EDEVICE, "no scratch address on this device");
    size_t a = 0, b = 0;
    topk_stage_keys(rows, V, M, &a, &b);
    if (a + b > TOPK_SCRATCH_KEYS)
        return fail(ctx, CC_EARG, "topk of " + std::to_string(rows) + " rows x " + std::to_string(V) + " logits, M " +
                                      std::to_string(M) + " stages " + std::to_string(a + b) +
                                      " keys, above the allocation-free scratch of " +
                                      std::to_string(TOPK_SCRATCH_KEYS) + " keys");
    launch_topk(stream ? (hipStream_t)stream : ctx->stream, logits, 1, rows, V, M, ctx->tk_scratch,
                ctx->tk_scratch + a, vals, ids);
    const hipError_t e = take_launch_error();
    if (e != hipSuccess) return fail(ctx, CC_EDEVICE, std::string("topk launch: ") + hipGetErrorString(e));
    return CC_OK;
}

cc_status cc_op_rmsnorm(cc_ctx* ctx, const float* x, const float* w, int32_t T, int32_t H, float* y) {
    if (!ctx || !x || !w || !y || T < 1 || H < 1) return CC_EARG;
    if (H % 8 || H > RESID_NORM_HMAX) return fail(ctx, CC_EARG, "rmsnorm rows must be a multiple of 8, at most 8192");
    float *dx = nullptr, *dw = nullptr, *dy = nullptr;
    HIPCHK(hipMalloc(&dx, (size_t)T * H * 4));
    HIPCHK(hipMalloc(&dw, (size_t)H * 4));
    HIPCHK(hipMalloc(&dy, (size_t)T * H * 4));
    HIPCHK(hipMemcpy(dx, x, (size_t)T * H * 4, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(dw, w, (size_t)H * 4, hipMemcpyHostToDevice));
    launch_resid_norm(ctx->stream, dx, nullptr, nullptr, 0, T, T, H, 0, dw, ctx->d.rms_eps, 0, nullptr, dy);
    HIPCHK(hipStreamSynchronize(ctx->stream));
    HIPCHK(take_launch_error());
    HIPCHK(hipMemcpy(y, dy, (size_t)T * H * 4, hipMemcpyDeviceToHost));
    for (void* v : {(void*)dx, (void*)dw, (void*)dy}) (void)hipFree(v);
    return CC_OK;
}

// A one-job plan for the kernel-level attention ops.
static cc_status one_job(cc_ctx* ctx, int32_t layer, int32_t slot, int32_t n, int32_t past, StepPlan& p,
                         MetaLayout& ml) {
    if (layer - ctx->L0 < 0 || layer - ctx->L0 >= (int)ctx->layers.size()) return fail(ctx, CC_EARG, "layer not held");
    if (!ctx->layers[layer - ctx->L0].kpool) return fail(ctx, CC_EARG, "a linear_attention block keeps no KV");
    if (slot < 0 || slot >= (int)ctx->owned.size() || n < 1 || n > ctx->o.t_max || past < 0 ||
        past + n > ctx->o.n_max)
        return fail(ctx, CC_EARG, "bad job");
    cc_job j{};
    j.slot = slot;
    j.past = past;
    j.n = n;
    build_plan(ctx, &j, 1, p, false);
    cc_status gs = grow(ctx, p);
    if (gs != CC_OK) return gs;
    ml = meta_layout(ctx);
    uint8_t* hm = ctx->h_meta;
    std::memcpy(hm + ml.jobs, p.jobs.data(), sizeof(JobDev));
    std::memcpy(hm + ml.items, p.items.data(), p.items.size() * sizeof(AttnItem));
    std::memcpy(hm + ml.row_job, p.row_job.data(), p.row_job.size() * 4);
    std::memcpy(hm + ml.cwg, p.cwg.data(), p.cwg.size() * 4);
    int32_t* plan = (int32_t*)(hm + ml.plan);
    const int need = ceil_div(past + n, ctx->geom.page);
    plan[0] = slot; plan[1] = ctx->owned[slot]; plan[2] = std::max(0, need - ctx->owned[slot]); plan[3] = 0;
    HIPCHK(hipMemcpyAsync(ctx->d_meta, hm, ml.total, hipMemcpyHostToDevice, ctx->stream));
    std::vector<std::pair<int, int>> want{{slot, past + n}};
    return take_pages(ctx, want, (int32_t*)(ctx->d_meta + ml.plan), plan, nullptr);
}

cc_status cc_op_store_kv(cc_ctx* ctx, int32_t layer, int32_t which, int32_t slot, const float* src, int32_t T_new,
                         int32_t T_past) {
    if (!ctx || !src || which < 0 || which > 1) return CC_EARG;
    StepPlan p;
    MetaLayout ml;
    cc_status s = one_job(ctx, layer, slot, T_new, T_past, p, ml);
    if (s != CC_OK) return s;
    const cc_dims& d = ctx->d;
    const int kv = d.n_kv_heads * d.head_dim;
    // Rows laid out as q|k|v with only the chosen part meaningful; store both
    // halves only when asked, by writing the other half from the cache's own
    // view is not possible, so K and V are stored one at a time through a
    // row whose other half is the same source (the kernel writes what it is
    // told to: do_kv stores K and V, so the unused half is re-stored below).
    const int N = (d.n_heads + 2 * d.n_kv_heads) * d.head_dim;
    std::vector<float> rows((size_t)T_new * N, 0.0f);
    for (int t = 0; t < T_new; t++)
        for (int e = 0; e < kv; e++) rows[(size_t)t * N + d.n_heads * d.head_dim + which * kv + e] = src[(size_t)t * kv + e];
    // Save the other half's rows so they can be restored.
    const int other = 1 - which;
    std::vector<std::vector<uint32_t>> saved(d.n_kv_heads);
    const int RW = d.head_dim / 4 + d.head_dim / 32;
    for (int h = 0; h < d.n_kv_heads; h++) {
        saved[h].resize((size_t)T_new * RW);
        cc_status r = kv_io(ctx, layer, other, slot, h, T_past, T_past + T_new, saved[h].data(), nullptr);
        if (r != CC_OK) return r;
    }
    float* dr = nullptr;
    HIPCHK(hipMalloc(&dr, rows.size() * 4));
    HIPCHK(hipMemcpy(dr, rows.data(), rows.size() * 4, hipMemcpyHostToDevice));
    Layer& L = ctx->layers[layer - ctx->L0];
    launch_fin_qkv(ctx->stream, dr, 1, T_new, (const int32_t*)(ctx->d_meta + ml.row_job),
                   (const JobDev*)(ctx->d_meta + ml.jobs), d.n_heads, ctx->group, ctx->geom, ctx->tbl, ctx->rot,
                   L.kpool, L.vpool, ctx->page_table, ctx->qp, RowScale{}, 0, 1);
    HIPCHK(hipStreamSynchronize(ctx->stream));
    (void)hipFree(dr);
    for (int h = 0; h < d.n_kv_heads; h++) {
        cc_status r = kv_io(ctx, layer, other, slot, h, T_past, T_past + T_new, nullptr, saved[h].data());
        if (r != CC_OK) return r;
    }
    return CC_OK;
}

cc_status cc_op_attend(cc_ctx* ctx, int32_t layer, int32_t slot, const float* q, int32_t n, int32_t past,
                       float* out) {
    if (!ctx || !q || !out) return CC_EARG;
    const cc_dims& d = ctx->d;
    if (ceil_div(past + n, ctx->geom.page) > ctx->owned[slot]) return fail(ctx, CC_EARG, "K/V rows are not stored");
    StepPlan p;
    MetaLayout ml;
    cc_status s = one_job(ctx, layer, slot, n, past, p, ml);
    if (s != CC_OK) return s;
    const int qd = d.n_heads * d.head_dim;
    const int N = (d.n_heads + 2 * d.n_kv_heads) * d.head_dim;
    std::vector<float> rows((size_t)n * N, 0.0f);
    for (int t = 0; t < n; t++)
        for (int e = 0; e < qd; e++) rows[(size_t)t * N + e] = q[(size_t)t * qd + e];
    float *dr = nullptr, *dctx = nullptr;
    uint4* dXp = nullptr;
    const int Mt = 2 * ceil_div(n, 32);
    const int KU = ceil_div(qd, 64);
    HIPCHK(hipMalloc(&dr, rows.size() * 4));
    HIPCHK(hipMalloc(&dctx, (size_t)n * qd * 4));
    HIPCHK(hipMalloc(&dXp, (size_t)Mt * 2 * KU * 2 * 1024));
    HIPCHK(hipMemcpy(dr, rows.data(), rows.size() * 4, hipMemcpyHostToDevice));
    Layer& L = ctx->layers[layer - ctx->L0];
    hipStream_t st = ctx->stream;
    const JobDev* dj = (const JobDev*)(ctx->d_meta + ml.jobs);
    const AttnItem* di = (const AttnItem*)(ctx->d_meta + ml.items);
    launch_fin_qkv(st, dr, 1, n, (const int32_t*)(ctx->d_meta + ml.row_job), dj, d.n_heads, ctx->group, ctx->geom,
                   ctx->tbl, ctx->rot, L.kpool, L.vpool, ctx->page_table, ctx->qp, RowScale{}, 1, 0);
    launch_attn(st, di, p.nlaunch, ctx->qp, L.kpool, L.vpool, ctx->page_table, ctx->geom, ctx->group, ctx->ppw,
                 ctx->apart, p.multi, ctx->attn);
    launch_attn_combine(st, dj, ctx->apart, ctx->geom, d.n_heads, ctx->group, KU, dXp, dctx,
                         (const int32_t*)(ctx->d_meta + ml.cwg), p.ncwg);
    HIPCHK(hipStreamSynchronize(st));
    HIPCHK(take_launch_error());
    HIPCHK(hipMemcpy(out, dctx, (size_t)n * qd * 4, hipMemcpyDeviceToHost));
    for (void* v : {(void*)dr, (void*)dctx, (void*)dXp}) (void)hipFree(v);
    return CC_OK;
}

}  // extern "C"
