// Launchers for the device kernels (kernels.hip). All take a stream and
// device pointers; shapes are validated by the caller (api.hip) before launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Tiled q8 weight (one 16-row x 64-column unit = 1 KiB of codes + 64 B of
// scales): codes [Nt][KU][64 lanes][16 B], byte b of lane l holds
// W[16t + l%16][64u + 32(b/8) + 8(l/16) + b%8] stored as q ^ 0x80; scales
// [Nt][KU][16][2] f16 for groups 2u, 2u+1 of row 16t + i.
struct QTensor {
    uint8_t* codes = nullptr;
    uint16_t* scales = nullptr;
    int N = 0, K = 0, Nt = 0, KU = 0;
};

// One pass's per-job table on the device (built on the host each step).
struct JobDev {
    int32_t slot, past, n, row0;   // rows row0 .. row0+n-1 of the pass
    int32_t qp_off;                // this job's Q operand base (uint4 units)
    int32_t mtq;                   // Q m-tiles (ceil(n*group/16))
    int32_t item0, nchunk;         // attention work items: item0 + kvh*nchunk + c
};

struct AttnItem {
    int32_t job, kvh, chunk, part; // part: float offset of the partial block
    int32_t mt;                    // query m-tile (16 rows rho = i*group + gi)
};

struct KVGeom {
    int nKV, D, ng, page, blk;     // blk: bytes per (page, kv head) block
    int max_pages;
};

void launch_gemm(hipStream_t st, const QTensor& w, const uint4* Xp, float* out, int M,
                 int splits, int nt);
void launch_prep_rows(hipStream_t st, const float* x, int ldx, int M, int Mpad, int K, int KU,
                      uint4* Xp);
void launch_rmsnorm_prep(hipStream_t st, const float* x, const int32_t* rows, int M, int Mpad,
                         int H, int KU, const float* w, float eps, uint4* Xp, float* y);
void launch_fin_residual(hipStream_t st, float* x, const float* part, int splits, int M, int H,
                         int round, const float* w, float eps, int KU, uint4* Xp, int Mpad);
void launch_fin_swiglu(hipStream_t st, const float* part, int splits, int M, int Mpad, int F,
                       int KU, uint4* Xp);
void launch_fin_qkv(hipStream_t st, const float* part, int splits, int M, const int32_t* row_job,
                    const JobDev* jobs, int nH, int group, const KVGeom& g, const float* tbl,
                    int rot, uint8_t* kpool, uint8_t* vpool, const uint32_t* page_table,
                    uint4* Qp, float* qkv_out, int do_q, int do_kv);
void launch_attn(hipStream_t st, const AttnItem* items, int nitems, const JobDev* jobs,
                 const uint4* Qp, const uint8_t* kpool, const uint8_t* vpool,
                 const uint32_t* page_table, const KVGeom& g, int group, float* part);
void launch_attn_combine(hipStream_t st, const JobDev* jobs, int njobs, const AttnItem* items,
                         const float* part, const KVGeom& g, int nH, int group, int M, int Mpad,
                         int KU, uint4* Xp, float* ctx_out);
void launch_embed(hipStream_t st, const int32_t* ids, const uint16_t* hidden, int T, const QTensor& wte,
                  float* x);
void launch_topk(hipStream_t st, const float* logits, int rows, int V, int M, uint64_t* a,
                 uint64_t* b, float* vals, uint32_t* ids);
void launch_round_f16(hipStream_t st, float* a, int64_t n);
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
void launch_tile_q8(hipStream_t st, const int8_t* codes, const uint16_t* scales, int N, int K,
                    int group, const QTensor& w, int row_tile0);
hipError_t take_launch_error();
void launch_resid_norm(hipStream_t st, float* x, const int32_t* rows, const float* part, int splits, int M,
                       int Mpad, int H, int round, const float* w, float eps, int KU, uint4* Xp, float* y,
                       float* ssq);
void launch_attn2(hipStream_t st, const AttnItem* items, int nitems, const JobDev* jobs, const uint4* Qp,
                  const uint8_t* kpool, const uint8_t* vpool, const uint32_t* page_table, const KVGeom& g, int group,
                  int ppw, float* part);
void launch_attn_combine2(hipStream_t st, const JobDev* jobs, int njobs, const AttnItem* items, const float* part,
                          const KVGeom& g, int nH, int group, int KU, uint4* Xp, float* ctx_out,
                          const int32_t* wg_job, int nwg);
void launch_sum_splits(hipStream_t st, const float* part, int splits, int M, int N, float* out);
void launch_to_half_bits(hipStream_t st, const float* x, int64_t n, uint16_t* out);
