// Launchers for the device kernels (kernels.hip). All take a stream and
// device pointers; shapes are validated by the caller (api.hip) before launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// q8 weight in matmul stream order. A tile is 16 rows x 64 columns of K (a
// "unit"); tiles pair up (t, t^1). K units split into P planes, plane r
// covering units [r*KU/P, (r+1)*KU/P) (at most LX_UNITS each; P from
// lx_planes_for when the tensor is allocated). For each
// plane, then each tile pair, then each unit of the plane, one record of
// LX_REC bytes:
//   [nt*1024 + lane*16 + b]  code of W[16t + lane%16][64u + 32(b/8) + 8(lane/16) + b%8]
//                            stored as q ^ 0x80 (t = 2*pair + nt)
//   [2048 + c*8 + nt*4 + h*2] f16 scale of row 16t + c, group 2u + h
// so the matmul reads each workgroup's weights as one forward stream.
constexpr int LX_UNITS = 20;     // K units whose activations one workgroup keeps in LDS
constexpr int LX_REC = 2176;     // bytes per (tile pair, unit) record

struct QTensor {
    uint8_t* codes = nullptr;    // records, Nt*KU*1088 bytes
    int N = 0, K = 0, Nt = 0, KU = 0, P = 1;
    // Scale format of the records' 128-byte scale block: 0 = one f16 per
    // row and 32-wide group (two per unit), 1 = one f32 per row and 64-wide
    // unit (a converter checkpoint's group-64 f32 scales, kept exactly).
    int f32s = 0;
    int up_f16 = 0, up_f32 = 0;  // parts uploaded in each format since the last fill
};

__host__ __device__ inline int lx_plane_start(int r, int KU, int P) { return (r * KU) / P; }
__host__ __device__ inline int lx_planes(int KU) { return (KU + LX_UNITS - 1) / LX_UNITS; }
// Byte offset of the record holding tile t, unit u.
__host__ __device__ inline size_t lx_record(int t, int u, int KU, int P, int Nt) {
    int r = (u * P) / KU;
    while (r + 1 < P && lx_plane_start(r + 1, KU, P) <= u) r++;
    while (r > 0 && lx_plane_start(r, KU, P) > u) r--;
    const int ua = lx_plane_start(r, KU, P), len = lx_plane_start(r + 1, KU, P) - ua;
    return ((size_t)ua * (Nt / 2) + (size_t)(t >> 1) * len + (size_t)(u - ua)) * LX_REC;
}

// One pass's per-job table on the device (built on the host each step).
struct JobDev {
    int32_t slot, past, n, row0;   // rows row0 .. row0+n-1 of the pass
    int32_t qp_off;                // this job's Q operand base (uint4 units)
    int32_t mtq;                   // Q m-tiles (ceil(n*group/16))
    int32_t item0, nchunk;         // attention work items: item0 + kvh*nchunk + c
    int32_t snap;                  // a verify: linear blocks snapshot their state
    int32_t keep;                  // >= 0: roll back to the snapshot, re-run `keep` rows
};

// One attention work item carries its job's fields itself (32 bytes, one
// scalar load), so a wave reaches its page table without a second
// dependent load.
struct AttnItem {
    int32_t slot, past, n;         // the job's session and rows
    int32_t mt;                    // query m-tile (16 rows rho = i*group + gi)
    int32_t qb;                    // Q operand base of (kv head, m-tile), uint4 units
    int32_t part;                  // float offset of the partial block
    int32_t kvh, p0;               // kv head, first page of the chunk
};

// A job as the host hands it to the device packer (k_pack): the pass's rows
// are packed in job order from these alone.
struct PackJob {
    int32_t slot, past, n, sampled;
    int32_t snap, keep;
};
// What the packer needs of the pass's geometry: kv heads, q heads per kv
// head, Q operand groups per head (ng), head_dim, pages per attention work
// item, and whether the pass reaches the head (its sampled rows).
constexpr int PACK_MAX_JOBS = 1024;   // jobs one pass may pack
struct PackGeom {
    int nKV, group, ng, D, ppw, page, head;
};

struct KVGeom {
    int nKV, D, ng, page, blk;     // blk: bytes per (page, kv head) block
    int max_pages;
};

constexpr int RESID_NORM_HMAX = 8192;
// rmsnorm's per-row factor 1/sqrt(ss/H + eps), from the slices' partial sums
// of squares ssp[m*RW_SMAX + s], s < nsl (added in slice order). With ssp
// null the factor is 1.
constexpr int RW_THREADS = 128, RW_SMAX = RESID_NORM_HMAX / 4 / RW_THREADS;
struct RowScale {
    const float* ssp = nullptr;
    int nsl = 0, H = 1;
    float eps = 0.f;
};

// Y planes: out[(r*M + m)*N + n], r < gemm_planes(w, M, ncu).
// Xp holds xp_mtiles m-tiles (16 rows each) of the operand; M > 32 reads
// those past M only as zeros.
void launch_gemm(hipStream_t st, const QTensor& w, const uint4* Xp, int xp_mtiles, float* out, int M, int ncu);
// The partial planes launch_gemm writes for w at M rows, which its consumers
// add in plane order: w.P, or 1 when the matmul adds them itself.
int gemm_planes(const QTensor& w, int M, int ncu);
int lx_groups(const QTensor& w, int ncu);
int lx_planes_for(int N, int K, int ncu);
void launch_prep_rows(hipStream_t st, const float* x, int ldx, int M, int Mpad, int K, int KU,
                      uint4* Xp);
void launch_fin_swiglu(hipStream_t st, const float* part, int splits, int M, int Mpad, int F,
                       int KU, uint4* Xp, const RowScale& rs);
// A hybrid checkpoint's full-attention extras (web/model/model.js:368-410):
// q_norm / k_norm (rmsnorm over each head's D values, applied before RoPE)
// and the output gate's projection, whose rows follow v in the fused q|k|v
// matmul and go to `gate` [M][nH*D] (times the row factor).
struct QkExtras {
    const float* qn = nullptr;
    const float* kn = nullptr;
    float eps = 0.f;
    float* gate = nullptr;
};
void launch_fin_qkv(hipStream_t st, const float* part, int splits, int M, const int32_t* row_job,
                    const JobDev* jobs, int nH, int group, const KVGeom& g, const float* tbl,
                    int rot, uint8_t* kpool, uint8_t* vpool, const uint32_t* page_table,
                    uint4* Qp, const RowScale& rs, int do_q, int do_kv, const QkExtras& ex = QkExtras{});

// Gated DeltaNet (web/model/kernels.js:1531-1839) over packed jobs. Columns of
// the fused projection (planes of N = 2*keyDim + 2*valueDim + 2*nVp): q, k, v
// (the conv channels, convDim = 2*keyDim + valueDim), z, b (nV, padded to
// nVp), a (nV, padded). `lraw` rows [M][LinGeom::W] hold the conv outputs
// (after SiLU), then z, b, a.
// A session's state (stride `sstride` floats, session `slot`):
//   block 0 (current) and block 1 (snapshot), `blk` floats each:
//     S [nV][Dk][Dv], then the conv ring [K-1][convDim] at `hist_off`;
//   at `rep_off`, a verify's rows [LIN_SPEC_ROWS][rep_w]: raw q|k|v
//     (convDim), conv outputs (convDim), b (nV), a (nV).
// `lrep` [jobs][LIN_SPEC_ROWS][lrep_w]: the rows a rollback re-runs, conv
// outputs then b, a, copied out before a verify overwrites them.
constexpr int LIN_SPEC_ROWS = 8;   // SPEC_COLS (web/split.js:273)
struct LinGeom {
    int nK = 0, nV = 0, Dk = 0, Dv = 0, K4 = 4, group = 1;
    int keyDim = 0, valueDim = 0, convDim = 0, nVp = 0;
    int W = 0;          // convDim + valueDim + 2*nV
    int N = 0;          // fused projection rows
    size_t blk = 0, hist_off = 0, rep_off = 0, sstride = 0;
    int rep_w = 0, lrep_w = 0;
};
constexpr int LIN_CONV_K = 4;
void launch_lin_conv(hipStream_t st, const float* part, int splits, int M, int njobs, const JobDev* jobs,
                     const RowScale& rs, const float* conv, const LinGeom& lg, float* state, float* lraw,
                     float* lrep);
// The conv parallel over rows, for a pass with a long job; `lring`
// [jobs][K-1][convDim] scratch.
constexpr int LIN_SEQ_ROWS = 16;   // longest job the one-thread-per-channel conv walks
void launch_lin_conv_rows(hipStream_t st, const float* part, int splits, int M, int njobs, const int32_t* row_job,
                          const JobDev* jobs, const RowScale& rs, const float* conv, const LinGeom& lg, float* state,
                          float* lraw, float* lrep, float* lring);
void launch_gdn(hipStream_t st, const float* lraw, const float* lrep, int njobs, const JobDev* jobs,
                const float* gp, const LinGeom& lg, float* state, float* core);
// RMSNormGated per (row, value head) with the gated_norm weight, times
// silu(z), into the out_proj operand (K = valueDim).
void launch_lin_norm(hipStream_t st, const float* core, const float* lraw, const float* gnorm, float eps,
                     int M, const LinGeom& lg, int KU, uint4* Xp);
// round: the trunk's rows are rounded to f16 (stage.js:1365-1370); the MTP
// head's draft embedding is not (model.js:545). An id past wte.N reads zero.
void launch_embed(hipStream_t st, const int32_t* ids, const uint16_t* hidden, int T, const QTensor& wte,
                  float* x, int round = 1);
void launch_gather_rows(hipStream_t st, const float* x, const float* alt, const int32_t* src, int T, int H,
                        float* rows);
void launch_topk(hipStream_t st, const float* logits, int planes, int rows, int V, int M, uint64_t* a,
                 uint64_t* b, float* vals, uint32_t* ids);
void launch_round_f16(hipStream_t st, float* a, int64_t n);
void launch_ids_col0(hipStream_t st, const uint32_t* ids, int rows, int stride, int32_t* out);
// Runner.#pass's packing (web/model/stage.js:1319-1346) on the device: from
// `njobs` PackJobs (each past advanced by `step`), the job table, the
// attention work items (kv head, m-tile, chunk of ppw pages; chunk fastest),
// row -> job, the sampled rows and the combine's (job, kv head, m-tile)
// triples, in the order the host planner writes them.
void launch_pack(hipStream_t st, const PackJob* in, int njobs, int step, const PackGeom& g, JobDev* jobs,
                 AttnItem* items, int32_t* row_job, int32_t* head_rows, int32_t* cwg);
// The keys launch_topk stages for (rows, V, M): a_keys for its first buffer,
// b_keys for its second.
void topk_stage_keys(int rows, int V, int M, size_t* a_keys, size_t* b_keys);
// The allocation-free top-k's scratch: a static device array of
// TOPK_SCRATCH_KEYS keys (4 MiB) per GPU. topk_scratch_setup looks up its
// address on `device` (which must be current) once, and returns it.
constexpr size_t TOPK_SCRATCH_KEYS = (size_t)1 << 19;
constexpr int TOPK_SCRATCH_DEVICES = 64;
hipError_t topk_scratch_setup(int device, uint64_t** out);
void launch_alloc_pages(hipStream_t st, const int32_t* plan, int njobs, const uint32_t* free_stack,
                        int top, uint32_t* page_table, int max_pages);
void launch_release_pages(hipStream_t st, int slot, int owned, uint32_t* free_stack, int top,
                          const uint32_t* page_table, int max_pages);
void launch_gen_q8(hipStream_t st, const QTensor& w, int row_tile0, int N, int K, uint64_t seed,
                   uint64_t stream);
void launch_fill(hipStream_t st, float* p, int64_t n, float v);
void launch_fill_kv(hipStream_t st, uint8_t* pool, const uint32_t* page_table, int slot, int tokens,
                    const KVGeom& g, uint64_t seed, uint64_t stream, uint64_t key, int which);
void launch_kv_to_ref(hipStream_t st, const uint8_t* pool, const uint32_t* page_table, int slot,
                      int head, int t0, int t1, const KVGeom& g, int which, uint32_t* out);
void launch_kv_from_ref(hipStream_t st, uint8_t* pool, const uint32_t* page_table, int slot,
                        int head, int t0, int t1, const KVGeom& g, int which, const uint32_t* in);
// scales: f16 [N, ceil(K/32)] when w.f32s == 0, f32 [N, ceil(K/64)] when 1.
void launch_tile_q8(hipStream_t st, const int8_t* codes, const void* scales, int N, int K, const QTensor& w,
                    int row_tile0);
hipError_t take_launch_error();
// Residual step (planes added in order, optional f16 round) and rmsnorm into
// the operand Xp or rows y, one workgroup per row; H % 8 == 0, H <= 8192.
// Residual step and the next matmul's operand x*w (rmsnorm without its row
// factor, which the matmul's consumer applies: RowScale), over (slice, row)
// workgroups; H % 64 == 0. With w null only the residual step runs.
void launch_resid_w(hipStream_t st, float* x, const float* part, int splits, int M, int Mpad, int H, int round,
                    const float* w, int KU, uint4* Xp, float* ssp);
void launch_resid_norm(hipStream_t st, float* x, const int32_t* rows, const float* part, int splits, int M,
                       int Mpad, int H, int round, const float* w, float eps, int KU, uint4* Xp, float* y);
// The attention launches of one stream: the CU count and a pair of device
// counters (zero at the start) from which launches a little over one round
// of workgroups hand out their last blocks; seq counts the launches.
struct AttnSched {
    uint32_t* ctr = nullptr;   // 2 counters
    uint32_t seq = 0;
    int ncu = 0;
};
void launch_attn(hipStream_t st, const AttnItem* items, int nitems, const uint4* Qp,
                  const uint8_t* kpool, const uint8_t* vpool, const uint32_t* page_table, const KVGeom& g, int group,
                  int ppw, float* part, int multi, AttnSched& sc);
// `gate` (a hybrid checkpoint's, [rows][nH*D], or null): the output is
// multiplied by sigmoid(gate) before it becomes the o_proj operand
// (web/model/kernels.js:1822-1839 sigmoid_mul).
void launch_attn_combine(hipStream_t st, const JobDev* jobs, const float* part, const KVGeom& g, int nH, int group,
                         int KU, uint4* Xp, float* ctx_out, const int32_t* wg_job, int nwg,
                         const float* gate = nullptr);
void launch_sum_splits(hipStream_t st, const float* part, int splits, int M, int N, float* out);
void launch_to_half_bits(hipStream_t st, const float* x, int64_t n, uint16_t* out);
