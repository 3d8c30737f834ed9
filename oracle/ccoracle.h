/* ccoracle.h — CPU restatement of the reference's batched ragged decode pass.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * library in chattorrent_amd/. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker or the
 * timed CPU baseline — never as a product path or a fallback.
 *
 * Every function restates one reference kernel's arithmetic, in the order the
 * reference's WGSL performs it, with plain IEEE f32 (compiled with
 * -ffp-contract=off so no product is fused into an FMA the reference does not
 * write). The file:line each follows is cited at the definition.
 */
#ifndef CCORACLE_H
#define CCORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* --- f16 (web/f16.js, kernels.js round_f16) --- */
uint16_t orc_half_bits(float x);
float    orc_half_value(uint16_t h);
void     orc_to_f16(const float* x, uint16_t* out, int64_t n);
void     orc_from_f16(const uint16_t* h, float* out, int64_t n);
void     orc_round_f16(float* a, int64_t n);

/* --- deterministic synthetic inputs (shared bit-for-bit with the device) --- */
uint64_t orc_rng(uint64_t seed, uint64_t stream, uint64_t i);
void orc_gen_q8(uint64_t seed, uint64_t stream, int64_t N, int64_t K, int group,
                int8_t* codes, uint16_t* scales_f16);
void orc_gen_normal_f16(uint64_t seed, uint64_t stream, int64_t n, uint16_t* out);
void orc_gen_ids(uint64_t seed, uint64_t stream, int64_t n, int vocab, int32_t* out);
uint16_t orc_gen_scale_f16(uint64_t seed, uint64_t stream, uint64_t i,
                           double lo, double hi);
void orc_gen_kv(uint64_t seed, uint64_t stream, uint64_t key, int t0, int tokens, int nKV,
                int D, int8_t* codes, float* scales);
void orc_fill_kv_paged(uint64_t seed, uint64_t stream, uint64_t key, int tokens, int nKV, int D,
                       int page, const uint32_t* pages, uint32_t* cache);

/* --- kernels (web/model/kernels.js) --- */
void orc_matmul_q8(const float* X, int M, int K, const int8_t* W, const float* S,
                   int N, int group, float* Y);
void orc_gather_embed_q8(const int32_t* ids, int T, int H, const int8_t* wte,
                         const float* S, int group, float* out);
void orc_rmsnorm(const float* x, const float* w, float* y, int T, int H, float eps);
void orc_rope_table(int rot, double theta, const double* scaling, int cap, float* tbl);
void orc_rope(float* buf, int nH, int T, int rot, int D, int T_past, const float* tbl);
void orc_store_kv(const float* src, uint32_t* cache, int T_new, int T_past, int page,
                  int nKV, int D, int rot, const uint32_t* pages, const float* tbl);
void orc_qk_scores(const float* Q, const uint32_t* K, float* scores, int T_new, int T_act,
                   int page, int D, int nH, int group, const uint32_t* pages, int r0, int T_q);
void orc_causal_softmax(float* scores, int T_new, int T_act, int T_past, int nH);
void orc_attn_av(const float* scores, const uint32_t* V, float* out, int T_new, int T_act,
                 int page, int D, int nH, int group, const uint32_t* pages, int r0, int T_q);
void orc_silu_mul(const float* g, const float* u, float* out, int64_t n);
void orc_add_inplace(float* a, const float* b, int64_t n);
void orc_topk(const float* row, int V, int M, float* vals, uint32_t* ids);

#ifdef __cplusplus
}
#endif
#endif
