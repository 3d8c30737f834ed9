// Device kernels of the MI355X (gfx950) batched ragged decode pass.
//
// Reference counterparts (l-wn/ChatTorrent, web/model/kernels.js) are cited
// per kernel. The design is MI355X-first: q8 projections run on MFMA
// (v_mfma_f32_16x16x32_f16) with the int8 codes dequantised exactly to f16 in
// registers and the f32 activations split into an f16 hi/lo pair, so each
// 32-wide quantisation group is one MFMA pair followed by one scale FMA per
// output; attention streams each chat's int8 pages once per kv head for the
// whole GQA group, also on MFMA; element-wise work is fused into the
// reduction ("finish") kernels that feed the next projection its operand.
#include "common.h"
#include "kernels.h"
#include <algorithm>
#include <mutex>
#include <type_traits>

// The first launch error since the last take_launch_error(); cc_step and the
// other entry points report it as CC_EDEVICE after their synchronisation.
static hipError_t g_launch_error = hipSuccess;
hipError_t take_launch_error() {
    hipError_t e = g_launch_error;
    g_launch_error = hipSuccess;
    return e;
}
#define CHECK_LAUNCH()                                                       \
    do {                                                                     \
        hipError_t e_ = hipGetLastError();                                   \
        if (e_ != hipSuccess && g_launch_error == hipSuccess) g_launch_error = e_; \
    } while (0)

// ===================================================================== GEMM ===
// Y[M, N] = X[M, K] . W[N, K]^T for a q8 W in record order (kernels.h) and an
// activation operand Xp prepared by the prep/finish kernels:
//   Xp[((mt*G2 + g)*2 + hl)*64 + lane] = 8 f16 of X[16mt + lane%16][32g + 8(lane/16) ..]
// (hl = 0: hi part, 1: lo part scaled by 2^11 (split_hilo_x), which meets the
// weights scaled by 2^-11; G2 = 2*KU groups, zero beyond K).
// Reference: matmul_gemv_q8 / matmul_gemv_rows_q8 / matmul_rows_q8 /
// matmul_tiled_q8 (web/model/kernels.js:449-804): per group, acc += scale * dot(x, q).
//
// Workgroup g (8 waves) serves plane r = g % P and a contiguous block of tile
// pairs; it first copies the plane's activations (MT m-tiles x <= LX_UNITS
// units, <= 160 KiB) into LDS, so the waves' only global loads are the weight
// records, which stream LX_R - 1 steps ahead. A "step" is one (pair, unit)
// record; the workgroup's steps are split evenly over its waves in record
// order, so each wave reads one forward run of memory. A pair cut between
// waves is finished by the wave holding its first units, adding the others'
// parts in unit order; the parts meet in LDS once every wave is past its last
// step (the activations are dead by then). Every split point depends on N, K
// and the CU count, never on M, so a row's result is the same in any batch.
// Output: plane r to out[(r*M + m)*N + n]; consumers add planes 0..P-1 in order
// (gemm_planes: one plane when k_gemm_tm_sum has added them).
constexpr int LX_WAVES = 8;
// The weight ring: one record in flight a wave ahead of the one computed.
// Measured at configs[2]: two or three records ahead made the pass 4-6%
// slower (more requests outstanding across the GPU's 2048 waves), none ahead
// 13% slower.
constexpr int LX_R = 2;

typedef __attribute__((address_space(3))) void lds_void_t;

// The scale of half-group h (K columns 32h .. 32h+31 of the unit) of one
// tile row, from the row's 32-bit word in the record's scale block: an f16
// per 32-wide group (h = 0 in the low half), or one f32 per 64-wide unit
// that both halves share (QTensor::f32s).
template <bool F32S>
__device__ static inline float rec_scale(uint32_t word, int h) {
    if constexpr (F32S) {
        (void)h;
        return __builtin_bit_cast(float, word);
    } else {
        const uint16_t s16 = h ? (uint16_t)(word >> 16) : (uint16_t)(word & 0xffffu);
        return (float)__builtin_bit_cast(_Float16, s16);
    }
}

template <int MT, bool F32S>
__global__ __launch_bounds__(64 * LX_WAVES) void k_gemm_lx(const uint8_t* __restrict__ Wr,
                                                           const uint4* __restrict__ Xp, float* __restrict__ out,
                                                           int KU, int M, int N, int Nt, int P, int Gm) {
    constexpr int NT = 2, R = LX_R, PW = R - 1, WAVES = LX_WAVES;
    extern __shared__ __attribute__((aligned(1024))) u32x4 xs[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = blockIdx.x % P, j = blockIdx.x / P;
    const int ua = lx_plane_start(r, KU, P), len = lx_plane_start(r + 1, KU, P) - ua;
    const int npairs = Nt / NT;
    const int p0 = (j * npairs) / Gm, p1 = ((j + 1) * npairs) / Gm;
    const int steps = (p1 - p0) * len;
    const int sw0 = (wave * steps) / WAVES, sw1 = ((wave + 1) * steps) / WAVES;
    const int nst = sw1 - sw0;
    const int mt0 = blockIdx.y * MT;
    const int G2 = 2 * KU;
    const auto rw = __builtin_amdgcn_make_buffer_rsrc((void*)Wr, 0, 0x7fffffff, 0x00020000);
    const auto rx = __builtin_amdgcn_make_buffer_rsrc((void*)Xp, 0, 0x7fffffff, 0x00020000);
    // Plane r's rows only: stores of rows >= M fall outside and are dropped.
    const auto ro = __builtin_amdgcn_make_buffer_rsrc((void*)(out + (size_t)r * M * N), 0, M * N * 4, 0x00020000);
    const int vw = lane * 16, vs = NT * 1024 + (lane & 15) * NT * 4;
    const int vo = (4 * (lane >> 4) * N + (lane & 15)) * 4;
    const int rec0 = ua * npairs + p0 * len;

    u32x4 w[R][NT];
    uint32_t s[R][NT];
    int sl = sw0;   // next step to load; stays on the last one past the end
    auto load_w = [&](u32x4 (&wv)[NT], uint32_t (&sv)[NT]) {
        const int off = (rec0 + sl) * LX_REC;
        wv[0] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, off, 2);
        wv[1] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, off + 1024, 2);
        const auto sc = __builtin_amdgcn_raw_buffer_load_b64(rw, vs, off, 0);
        sv[0] = sc[0];
        sv[1] = sc[1];
        if (sl + 1 < sw1) sl++;
    };
    if (nst > 0) {
#pragma unroll
        for (int i = 0; i < PW; i++) load_w(w[i], s[i]);
    }
    // Activations of this plane into LDS: block (u, mt, q) of 1 KiB, q = 2h + hl.
    {
        const int nblk = len * MT * 4;
        for (int b = wave; b < nblk; b += WAVES) {
            const int u = b / (MT * 4), mt = (b / 4) % MT, q = b % 4;
            const int src = ((mt0 + mt) * G2 + 2 * (ua + u) + (q >> 1)) * 2 + (q & 1);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(xs + b * 64), 16, vw, src * 1024, 0, 0);
        }
    }
    float4_t acc[MT][NT], tail[MT][NT];   // tail: this wave's part of a pair begun in an earlier wave
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[mt][nt] = tail[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    auto compute = [&](const u32x4 (&wc)[NT], const uint32_t (&sc)[NT], int u) {
        u32x4 xv[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int q = 0; q < 4; q++) xv[mt][q] = xs[((u * MT + mt) * 4 + q) * 64 + lane];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            half8_t b[NT];
            float scale[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                b[nt] = h ? dequant8_biased(wc[nt][2], wc[nt][3]) : dequant8_biased(wc[nt][0], wc[nt][1]);
                scale[nt] = rec_scale<F32S>(sc[nt], h);
            }
            // hi then lo into one partial per output, then one scale FMA
            float4_t pp[MT][NT];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    pp[mt][nt] = mfma16x16x32(__builtin_bit_cast(half8_t, xv[mt][2 * h]), b[nt],
                                              float4_t{0.f, 0.f, 0.f, 0.f});
            half8_t bl[NT];   // the lo half carries 2^11 x its remainder
#pragma unroll
            for (int nt = 0; nt < NT; nt++) bl[nt] = lo_weight8(b[nt]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    pp[mt][nt] = mfma16x16x32(__builtin_bit_cast(half8_t, xv[mt][2 * h + 1]), bl[nt], pp[mt][nt]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        acc[mt][nt][e] = __builtin_fmaf(scale[nt], pp[mt][nt][e], acc[mt][nt][e]);
        }
    };
    auto store_plane = [&](int pair) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int tile = (p0 + pair) * NT + nt;
            if (tile * 16 >= N) continue;
            // columns past N of a partial tile would land in the next row
            if (tile * 16 + 16 > N && tile * 16 + (lane & 15) >= N) continue;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float v = acc[mt][nt][e];
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ro,
                                                          vo + (((mt0 + mt) * 16 + e) * N + tile * 16) * 4, 0, 0);
                }
        }
    };
    int pc = 0, uc = 0;   // (pair, unit) of the step being computed
    if (nst > 0) {
        pc = sw0 / len;
        uc = sw0 - pc * len;
    }
    bool head_open = false, has_tail = false;
    // After a pair's last unit (or this wave's last step) its partial goes to
    // `out` (whole pair), to `tail` (pair began in an earlier wave), or stays
    // in acc (pair goes on in later waves).
    auto finish_step = [&](int st) {
        if (uc == len - 1 || st == sw1 - 1) {
            if (pc * len < sw0) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) tail[mt][nt] = acc[mt][nt];
                has_tail = true;
            } else if ((pc + 1) * len <= sw1) {
                store_plane(pc);
            } else {
                head_open = true;
            }
            if (!head_open) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) acc[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
        if (++uc == len) {
            uc = 0;
            pc++;
        }
    };
    if (nst > 0) {
        int k = 0;
        for (; k + R <= nst; k += R) {
#pragma unroll
            for (int I = 0; I < R; I++) {
                load_w(w[(I + PW) % R], s[(I + PW) % R]);
                __builtin_amdgcn_sched_barrier(0);
                compute(w[I], s[I], uc);
                __builtin_amdgcn_sched_barrier(0);
                finish_step(sw0 + k + I);
            }
        }
        // At most PW steps remain, already in ring slots 0 .. PW-1.
#pragma unroll
        for (int I = 0; I < PW; I++) {
            if (k + I < nst) {
                compute(w[I], s[I], uc);
                finish_step(sw0 + k + I);
            }
        }
    }
    // Every wave is past its last step: the LDS activations are dead and hold
    // the cut parts now, one 1 KiB slot per (wave, m-tile, tile).
    __syncthreads();
    if (has_tail) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                xs[((wave * MT + mt) * NT + nt) * 64 + lane] = __builtin_bit_cast(u32x4, tail[mt][nt]);
    }
    __syncthreads();
    if (head_open) {
        const int pair = (sw1 - 1) / len, pe = (pair + 1) * len;
        for (int w2 = wave + 1; w2 < WAVES; w2++) {
            const int a2 = (w2 * steps) / WAVES, b2 = ((w2 + 1) * steps) / WAVES;
            if (a2 >= pe) break;
            if (b2 <= a2) continue;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const float4_t o = __builtin_bit_cast(float4_t, xs[((w2 * MT + mt) * NT + nt) * 64 + lane]);
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[mt][nt][e] = acc[mt][nt][e] + o[e];
                }
        }
        store_plane(pair);
    }
}

int lx_groups(const QTensor& w, int ncu) {
    const int per = std::max(1, std::min(ncu / w.P, w.Nt / 2));
    return w.P * per;
}

// K planes of an N x K q8 tensor: the fewest the LDS allows (lx_planes),
// doubled (up to 16, and to one unit a plane) while the workgroups the
// matmul launches (planes x column groups, lx_groups) would fill fewer than
// half the CUs. A small model's narrow matrices (30 tile pairs at
// SmolLM2's q|k|v) otherwise leave most CUs idle; a 27B or 8B layer fills
// them at the fewest planes and keeps those.
int lx_planes_for(int N, int K, int ncu) {
    const int KU = (K + 63) / 64, npairs = (N + 31) / 32;
    int P = lx_planes(KU);
    while (2 * P <= std::min(KU, 16) && 2LL * P * std::max(1, std::min(ncu / P, npairs)) <= ncu) P *= 2;
    return P;
}

template <int MT, bool F32S>
static void launch_lx(hipStream_t st, const QTensor& w, const uint4* Xp, float* out, int M, int ncu) {
    static bool attr = false;
    if (!attr) {
        attr = true;
        (void)hipFuncSetAttribute((const void*)k_gemm_lx<MT, F32S>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  LX_UNITS * MT * 4096);
    }
    const int G = lx_groups(w, ncu), Gm = G / w.P;
    const int lenmax = (w.KU + w.P - 1) / w.P;
    // the plane's activations, and afterwards the cut parts (1 KiB per wave, m-tile and tile)
    const size_t lds = std::max((size_t)lenmax * MT * 4096, (size_t)LX_WAVES * MT * 2 * 1024);
    dim3 grid(G, (M + 16 * MT - 1) / (16 * MT));
    hipLaunchKernelGGL((k_gemm_lx<MT, F32S>), grid, dim3(64 * LX_WAVES), lds, st, (const uint8_t*)w.codes, Xp, out,
                       w.KU, M, w.N, w.Nt, w.P, Gm);
}

// ------------------------------------------------- many rows (M > 32) ---
// Above 32 rows k_gemm_lx would stream every weight once per 32-row block.
// k_gemm_tm reuses each weight record across 64 rows instead: a workgroup
// serves plane r (the same planes as k_gemm_lx), TM_PAIRS tile pairs and 64
// rows (4 m-tiles); wave (h, i) computes rows 32h .. 32h+31 of pair i, so
// each record feeds two waves. The activations of one unit of K for the 64
// rows (16 KiB) are staged through registers into a double-buffered LDS
// block, one barrier a unit, while each wave streams its pair's records
// TM_R-1 units ahead (144 VGPRs: two waves a SIMD).
//
// Bits: a row's result is bit-identical to k_gemm_lx's at any M. Within a
// plane k_gemm_lx sums a pair's units in order but in segments, cut where
// its workgroup's steps are split between waves, and adds the segments in
// order; the cut points depend only on N, K and the CU count (lx_cuts), and
// k_gemm_tm folds its running sum at the same units. Each MFMA pair, scale
// FMA and addition is the same operation on the same operands.
constexpr int TM_MT = 4, TM_WAVES = 8, TM_PAIRS = 8, TM_R = 2;

// Unit offsets inside pair p (of a plane of `len` <= 32 units) where
// k_gemm_lx starts a new partial sum, as a bit mask: the wave boundaries of
// the lx workgroup holding p (workgroup j of Gm covers pairs
// [j*npairs/Gm, (j+1)*npairs/Gm)) that fall strictly inside the pair.
__device__ static inline uint32_t lx_cuts(int p, int npairs, int Gm, int len) {
    int j = (int)(((long long)p * Gm) / npairs);
    while (j > 0 && (int)(((long long)j * npairs) / Gm) > p) j--;
    while (j + 1 < Gm && (int)(((long long)(j + 1) * npairs) / Gm) <= p) j++;
    const int p0 = (int)(((long long)j * npairs) / Gm), p1 = (int)(((long long)(j + 1) * npairs) / Gm);
    const int steps = (p1 - p0) * len, s0 = (p - p0) * len;
    uint32_t m = 0;
#pragma unroll
    for (int w = 1; w < LX_WAVES; w++) {
        const int b = (w * steps) / LX_WAVES - s0;
        if (b > 0 && b < len) m |= 1u << b;
    }
    return m;
}

template <bool F32S>
__global__ __launch_bounds__(64 * TM_WAVES) void k_gemm_tm(const uint8_t* __restrict__ Wr,
                                                              const uint4* __restrict__ Xp, int xp_mtiles,
                                                              float* __restrict__ out, int KU, int M, int N, int Nt,
                                                              int P, int Gm) {
    constexpr int NT = 2, R = TM_R, PW = R - 1, MTL = TM_MT, MTW = MTL * TM_PAIRS / TM_WAVES;
    static_assert(MTW * TM_WAVES == MTL * TM_PAIRS, "waves cover pairs x m-tiles");
    __shared__ u32x4 xs[2][MTL * 4][64];   // two units: block (m-tile, q = 2h + hl) of 1 KiB
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int npairs = Nt / NT;
    // Workgroups b and b + 8 run on one XCD (dispatch is round-robin over the
    // XCDs, from an offset that varies by launch).
    // Each (plane, pair group) goes to one XCD, which runs its row blocks back
    // to back, so the row blocks after the first read its weight records from
    // that XCD's L2 instead of HBM. The order of workgroups changes no sums.
    const int nrb = (M + 16 * MTL - 1) / (16 * MTL), npg = (npairs + TM_PAIRS - 1) / TM_PAIRS;
    const int kx = blockIdx.x / 8;
    const int gx = (kx / nrb) * 8 + blockIdx.x % 8, gy = kx % nrb;
    if (gx >= P * npg) return;   // the grid is rounded up to whole XCD rounds
    const int r = gx % P, pb = gx / P;
    const int pair = pb * TM_PAIRS + wave % TM_PAIRS, mw = (wave / TM_PAIRS) * MTW;   // m-tiles mw .. mw+MTW-1
    const bool has = pair < npairs;
    const int ua = lx_plane_start(r, KU, P), len = lx_plane_start(r + 1, KU, P) - ua;
    const int mt0 = gy * MTL;
    const int G2 = 2 * KU;
    const auto rw = __builtin_amdgcn_make_buffer_rsrc((void*)Wr, 0, 0x7fffffff, 0x00020000);
    // activation m-tiles past the operand's allocation read zero
    const uint32_t xbytes = (uint32_t)min((unsigned long long)xp_mtiles * G2 * 2048ull, 0xffffffffull);
    const auto rx = __builtin_amdgcn_make_buffer_rsrc((void*)Xp, 0, xbytes, 0x00020000);
    const auto ro = __builtin_amdgcn_make_buffer_rsrc((void*)(out + (size_t)r * M * N), 0, M * N * 4, 0x00020000);
    const int vw = lane * 16, vs = NT * 1024 + (lane & 15) * NT * 4;
    const int vo = (4 * (lane >> 4) * N + (lane & 15)) * 4;
    const int rec0 = (ua * npairs + (has ? pair : 0) * len) * LX_REC;
    const uint32_t cuts = has ? lx_cuts(pair, npairs, Gm, len) : 0u;

    // this wave's share of a unit's activations: blocks BPW*wave .. +BPW-1
    constexpr int BPW = MTL * 4 / TM_WAVES;
    static_assert(BPW * TM_WAVES == MTL * 4, "activation blocks split evenly over the waves");
    u32x4 st[BPW];
    auto load_x = [&](int u) {
        const int Uk = ua + (u < len ? u : len - 1);
#pragma unroll
        for (int k = 0; k < BPW; k++) {
            const int b = BPW * wave + k, mt = b >> 2, q = b & 3;
            const int src = ((mt0 + mt) * G2 + 2 * Uk + (q >> 1)) * 2 + (q & 1);
            st[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, vw, src * 1024, 0);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int k = 0; k < BPW; k++) xs[buf][BPW * wave + k][lane] = st[k];
    };
    u32x4 w[R][NT];
    uint32_t sc[R][NT];
    auto load_w = [&](int u, u32x4 (&wv)[NT], uint32_t (&sv)[NT]) {
        const int off = rec0 + (u < len ? u : len - 1) * LX_REC;
        wv[0] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, off, 2);
        wv[1] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, off + 1024, 2);
        const auto s2 = __builtin_amdgcn_raw_buffer_load_b64(rw, vs, off, 0);
        sv[0] = s2[0];
        sv[1] = s2[1];
    };
    float4_t seg[MTW][NT], tot[MTW][NT];
#pragma unroll
    for (int mt = 0; mt < MTW; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) seg[mt][nt] = tot[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
    bool started = false;   // tot holds the first segment(s)

    load_x(0);
#pragma unroll
    for (int i = 0; i < PW; i++) load_w(i, w[i], sc[i]);
    store_x(0);
    load_x(1);
    __syncthreads();

    auto unit = [&](int u, const u32x4 (&wc)[NT], const uint32_t (&sv)[NT]) {
        const int buf = u & 1;
        // the unit k_gemm_lx begins a new partial sum at: fold the running one
        if ((cuts >> u) & 1u) {
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    if (started)
#pragma unroll
                        for (int e = 0; e < 4; e++) tot[mt][nt][e] = tot[mt][nt][e] + seg[mt][nt][e];
                    else
                        tot[mt][nt] = seg[mt][nt];
                    seg[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
                }
            started = true;
        }
        half8_t b[2][NT], bl[2][NT];   // bl: the lo half's fragment, 2^-11 b
        float scale[2][NT];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                b[h][nt] = h ? dequant8_biased(wc[nt][2], wc[nt][3]) : dequant8_biased(wc[nt][0], wc[nt][1]);
                bl[h][nt] = lo_weight8(b[h][nt]);
                scale[h][nt] = rec_scale<F32S>(sv[nt], h);
            }
        // per half-group, every m-tile's MFMA pair first and the scale FMAs
        // after them, so no FMA waits on the MFMA issued just before it; each
        // output's operations and their order are those of k_gemm_lx
#pragma unroll
        for (int h = 0; h < 2; h++) {
            u32x4 xv[MTW][2];
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int q = 0; q < 2; q++) xv[mt][q] = xs[buf][(mw + mt) * 4 + 2 * h + q][lane];
            float4_t pp[MTW][NT];
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    pp[mt][nt] = mfma16x16x32(__builtin_bit_cast(half8_t, xv[mt][0]), b[h][nt], float4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    pp[mt][nt] = mfma16x16x32(__builtin_bit_cast(half8_t, xv[mt][1]), bl[h][nt], pp[mt][nt]);
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int e = 0; e < 4; e++) seg[mt][nt][e] = __builtin_fmaf(scale[h][nt], pp[mt][nt][e], seg[mt][nt][e]);
        }
    };
    int u = 0;
    for (; u + R <= len; u += R) {
#pragma unroll
        for (int I = 0; I < R; I++) {
            load_w(u + I + PW, w[(I + PW) % R], sc[(I + PW) % R]);
            unit(u + I, w[I], sc[I]);
            // the next unit's activations go in the other buffer: every wave
            // finished reading it (one unit ago) before the last barrier
            store_x((I + 1) & 1);
            load_x(u + I + 2);
            __syncthreads();
        }
    }
    // at most PW units remain, their records in ring slots 0 .. PW-1
#pragma unroll
    for (int I = 0; I < PW; I++) {
        if (u + I < len) {
            unit(u + I, w[I], sc[I]);
            store_x((I + 1) & 1);
            load_x(u + I + 2);
            __syncthreads();
        }
    }
    if (!has) return;
#pragma unroll
    for (int mt = 0; mt < MTW; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            if (started)
#pragma unroll
                for (int e = 0; e < 4; e++) tot[mt][nt][e] = tot[mt][nt][e] + seg[mt][nt][e];
            else
                tot[mt][nt] = seg[mt][nt];
        }
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int tile = pair * NT + nt;
        if (tile * 16 >= N) continue;
        if (tile * 16 + 16 > N && tile * 16 + (lane & 15) >= N) continue;
#pragma unroll
        for (int mt = 0; mt < MTW; mt++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(tot[mt][nt][e]), ro,
                                                      vo + (((mt0 + mw + mt) * 16 + e) * N + tile * 16) * 4, 0, 0);
    }
}

// k_gemm_tm12: k_gemm_tm at twelve waves a workgroup (three a SIMD), each
// still one tile pair over the row block's 4 m-tiles, for matrices whose
// pair groups of twelve still give every CU a workgroup. The running sum of
// the segments already folded (k_gemm_tm's `tot`) lives in the wave's own
// LDS slot (8 KiB a wave) instead of 32 registers, which brings the kernel
// to 160 VGPRs: three waves a SIMD. A fold reads the slot, adds the segment
// and writes it back: the same additions in the same order, so every output
// keeps k_gemm_tm's (and k_gemm_lx's) bits. The staged activation blocks of
// a unit (16) are shared out over the twelve waves, one or two each.
constexpr int TM12_WAVES = 12;
template <bool F32S>
__global__ __launch_bounds__(64 * TM12_WAVES) void k_gemm_tm12(const uint8_t* __restrict__ Wr,
                                                              const uint4* __restrict__ Xp, int xp_mtiles,
                                                              float* __restrict__ out, int KU, int M, int N, int Nt,
                                                              int P, int Gm) {
    constexpr int NT = 2, R = TM_R, PW = R - 1, MTL = TM_MT, WV = TM12_WAVES;
    __shared__ u32x4 xs[2][MTL * 4][64];
    __shared__ float4_t tl[WV][MTL * NT][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int npairs = Nt / NT;
    const int nrb = (M + 16 * MTL - 1) / (16 * MTL), npg = (npairs + WV - 1) / WV;
    const int kx = blockIdx.x / 8;
    const int gx = (kx / nrb) * 8 + blockIdx.x % 8, gy = kx % nrb;
    if (gx >= P * npg) return;
    const int r = gx % P, pb = gx / P;
    const int pair = pb * WV + wave;
    const bool has = pair < npairs;
    const int ua = lx_plane_start(r, KU, P), len = lx_plane_start(r + 1, KU, P) - ua;
    const int mt0 = gy * MTL;
    const int G2 = 2 * KU;
    const auto rw = __builtin_amdgcn_make_buffer_rsrc((void*)Wr, 0, 0x7fffffff, 0x00020000);
    const uint32_t xbytes = (uint32_t)min((unsigned long long)xp_mtiles * G2 * 2048ull, 0xffffffffull);
    const auto rx = __builtin_amdgcn_make_buffer_rsrc((void*)Xp, 0, xbytes, 0x00020000);
    const auto ro = __builtin_amdgcn_make_buffer_rsrc((void*)(out + (size_t)r * M * N), 0, M * N * 4, 0x00020000);
    const int vw = lane * 16, vs = NT * 1024 + (lane & 15) * NT * 4;
    const int vo = (4 * (lane >> 4) * N + (lane & 15)) * 4;
    const int rec0 = (ua * npairs + (has ? pair : 0) * len) * LX_REC;
    const uint32_t cuts = has ? lx_cuts(pair, npairs, Gm, len) : 0u;
    constexpr int NB = MTL * 4, BPW = (NB + WV - 1) / WV;
    u32x4 st[BPW];
    auto load_x = [&](int u) {
        const int Uk = ua + (u < len ? u : len - 1);
#pragma unroll
        for (int k = 0; k < BPW; k++) {
            const int b = wave + k * WV, mt = b >> 2, q = b & 3;
            if (b < NB) {
                const int src = ((mt0 + mt) * G2 + 2 * Uk + (q >> 1)) * 2 + (q & 1);
                st[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, vw, src * 1024, 0);
            }
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int k = 0; k < BPW; k++) {
            const int b = wave + k * WV;
            if (b < NB) xs[buf][b][lane] = st[k];
        }
    };
    u32x4 w[R][NT];
    uint32_t sc[R][NT];
    auto load_w = [&](int u, u32x4 (&wv)[NT], uint32_t (&sv)[NT]) {
        const int off = rec0 + (u < len ? u : len - 1) * LX_REC;
        wv[0] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, off, 2);
        wv[1] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, off + 1024, 2);
        const auto s2 = __builtin_amdgcn_raw_buffer_load_b64(rw, vs, off, 0);
        sv[0] = s2[0];
        sv[1] = s2[1];
    };
    float4_t seg[MTL][NT];
#pragma unroll
    for (int mt = 0; mt < MTL; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) seg[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
    bool started = false;

    load_x(0);
#pragma unroll
    for (int i = 0; i < PW; i++) load_w(i, w[i], sc[i]);
    store_x(0);
    load_x(1);
    __syncthreads();

    auto fold = [&]() {
#pragma unroll
        for (int mt = 0; mt < MTL; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                float4_t t = seg[mt][nt];
                if (started) {
                    const float4_t o = tl[wave][mt * NT + nt][lane];
#pragma unroll
                    for (int e = 0; e < 4; e++) t[e] = o[e] + seg[mt][nt][e];
                }
                tl[wave][mt * NT + nt][lane] = t;
                seg[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
            }
        started = true;
    };
    auto unit = [&](int u, const u32x4 (&wc)[NT], const uint32_t (&sv)[NT]) {
        const int buf = u & 1;
        if ((cuts >> u) & 1u) fold();
        half8_t b[2][NT], bl[2][NT];
        float scale[2][NT];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                b[h][nt] = h ? dequant8_biased(wc[nt][2], wc[nt][3]) : dequant8_biased(wc[nt][0], wc[nt][1]);
                bl[h][nt] = lo_weight8(b[h][nt]);
                scale[h][nt] = rec_scale<F32S>(sv[nt], h);
            }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            u32x4 xv[MTL][2];
#pragma unroll
            for (int mt = 0; mt < MTL; mt++)
#pragma unroll
                for (int q = 0; q < 2; q++) xv[mt][q] = xs[buf][mt * 4 + 2 * h + q][lane];
            float4_t pp[MTL][NT];
#pragma unroll
            for (int mt = 0; mt < MTL; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    pp[mt][nt] = mfma16x16x32(__builtin_bit_cast(half8_t, xv[mt][0]), b[h][nt], float4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int mt = 0; mt < MTL; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    pp[mt][nt] = mfma16x16x32(__builtin_bit_cast(half8_t, xv[mt][1]), bl[h][nt], pp[mt][nt]);
#pragma unroll
            for (int mt = 0; mt < MTL; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int e = 0; e < 4; e++) seg[mt][nt][e] = __builtin_fmaf(scale[h][nt], pp[mt][nt][e], seg[mt][nt][e]);
        }
    };
    int u = 0;
    for (; u + R <= len; u += R) {
#pragma unroll
        for (int I = 0; I < R; I++) {
            load_w(u + I + PW, w[(I + PW) % R], sc[(I + PW) % R]);
            unit(u + I, w[I], sc[I]);
            store_x((I + 1) & 1);
            load_x(u + I + 2);
            __syncthreads();
        }
    }
#pragma unroll
    for (int I = 0; I < PW; I++) {
        if (u + I < len) {
            unit(u + I, w[I], sc[I]);
            store_x((I + 1) & 1);
            load_x(u + I + 2);
            __syncthreads();
        }
    }
    if (!has) return;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int tile = pair * NT + nt;
        if (tile * 16 >= N) continue;
        if (tile * 16 + 16 > N && tile * 16 + (lane & 15) >= N) continue;
#pragma unroll
        for (int mt = 0; mt < MTL; mt++) {
            float4_t t = seg[mt][nt];
            if (started) {
                const float4_t o = tl[wave][mt * NT + nt][lane];
#pragma unroll
                for (int e = 0; e < 4; e++) t[e] = o[e] + seg[mt][nt][e];
            }
#pragma unroll
            for (int e = 0; e < 4; e++)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(t[e]), ro,
                                                      vo + (((mt0 + mt) * 16 + e) * N + tile * 16) * 4, 0, 0);
        }
    }
}

// k_gemm_tm_sum: k_gemm_tm over every plane of its pairs and rows in one
// workgroup, unit by unit in K order. Each plane is finished as k_gemm_tm
// finishes it (the same segments and folds), and the finished planes are
// added in plane order into the one plane it writes: the sum every consumer
// forms from the P planes (in order from plane 0; those that pad with zero
// loads pad this sum the same way when P < 16), so the bits are the same,
// and the P-plane write and read are spared. For rows enough to fill the
// GPU without the K split (gemm_planes).
template <bool F32S>
__global__ __launch_bounds__(64 * TM_WAVES) void k_gemm_tm_sum(const uint8_t* __restrict__ Wr,
                                                              const uint4* __restrict__ Xp, int xp_mtiles,
                                                              float* __restrict__ out, int KU, int M, int N, int Nt,
                                                              int P, int Gm) {
    constexpr int NT = 2, R = TM_R, PW = R - 1, MTL = TM_MT, MTW = MTL * TM_PAIRS / TM_WAVES;
    static_assert(MTW * TM_WAVES == MTL * TM_PAIRS, "waves cover pairs x m-tiles");
    __shared__ u32x4 xs[2][MTL * 4][64];   // two units: block (m-tile, q = 2h + hl) of 1 KiB
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int npairs = Nt / NT;
    // Each pair group goes to one XCD, which runs its row blocks back to back
    // (the mapping of k_gemm_tm with one plane).
    const int nrb = (M + 16 * MTL - 1) / (16 * MTL), npg = (npairs + TM_PAIRS - 1) / TM_PAIRS;
    const int kx = blockIdx.x / 8;
    const int gx = (kx / nrb) * 8 + blockIdx.x % 8, gy = kx % nrb;
    if (gx >= npg) return;   // the grid is rounded up to whole XCD rounds
    const int pb = gx;
    const int pair = pb * TM_PAIRS + wave % TM_PAIRS, mw = (wave / TM_PAIRS) * MTW;   // m-tiles mw .. mw+MTW-1
    const bool has = pair < npairs;
    const int ua = 0, len = KU;   // every unit, planes in order
    const int mt0 = gy * MTL;
    const int G2 = 2 * KU;
    const auto rw = __builtin_amdgcn_make_buffer_rsrc((void*)Wr, 0, 0x7fffffff, 0x00020000);
    // activation m-tiles past the operand's allocation read zero
    const uint32_t xbytes = (uint32_t)min((unsigned long long)xp_mtiles * G2 * 2048ull, 0xffffffffull);
    const auto rx = __builtin_amdgcn_make_buffer_rsrc((void*)Xp, 0, xbytes, 0x00020000);
    const auto ro = __builtin_amdgcn_make_buffer_rsrc((void*)out, 0, M * N * 4, 0x00020000);
    const int vw = lane * 16, vs = NT * 1024 + (lane & 15) * NT * 4;
    const int vo = (4 * (lane >> 4) * N + (lane & 15)) * 4;
    const int pr0 = has ? pair : 0;
    // the load cursor (units are loaded in increasing order, PW ahead of
    // compute): the plane holding the next unit to load and its first record
    int lp = 0, lend = lx_plane_start(1, KU, P), lbase = 0, lrec = pr0 * lend * LX_REC;
    // the compute cursor: the plane being summed, its end and cut points
    int cp = 0, cbase = 0, cend = lend;
    uint32_t cuts = has ? lx_cuts(pair, npairs, Gm, cend) : 0u;

    // this wave's share of a unit's activations: blocks BPW*wave .. +BPW-1
    constexpr int BPW = MTL * 4 / TM_WAVES;
    static_assert(BPW * TM_WAVES == MTL * 4, "activation blocks split evenly over the waves");
    u32x4 st[BPW];
    auto load_x = [&](int u) {
        const int Uk = ua + (u < len ? u : len - 1);
#pragma unroll
        for (int k = 0; k < BPW; k++) {
            const int b = BPW * wave + k, mt = b >> 2, q = b & 3;
            const int src = ((mt0 + mt) * G2 + 2 * Uk + (q >> 1)) * 2 + (q & 1);
            st[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, vw, src * 1024, 0);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int k = 0; k < BPW; k++) xs[buf][BPW * wave + k][lane] = st[k];
    };
    u32x4 w[R][NT];
    uint32_t sc[R][NT];
    auto load_w = [&](int u, u32x4 (&wv)[NT], uint32_t (&sv)[NT]) {
        u = u < len ? u : len - 1;
        while (u >= lend) {   // the next plane: records [plane][pair][unit]
            lp++;
            lbase = lend;
            lend = lx_plane_start(lp + 1, KU, P);
            lrec = (lbase * npairs + pr0 * (lend - lbase)) * LX_REC;
        }
        const int off = lrec + (u - lbase) * LX_REC;
        wv[0] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, off, 2);
        wv[1] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, off + 1024, 2);
        const auto s2 = __builtin_amdgcn_raw_buffer_load_b64(rw, vs, off, 0);
        sv[0] = s2[0];
        sv[1] = s2[1];
    };
    float4_t seg[MTW][NT], tot[MTW][NT], sum[MTW][NT];
#pragma unroll
    for (int mt = 0; mt < MTW; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) seg[mt][nt] = tot[mt][nt] = sum[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
    bool started = false;   // tot holds the first segment(s)

    load_x(0);
#pragma unroll
    for (int i = 0; i < PW; i++) load_w(i, w[i], sc[i]);
    store_x(0);
    load_x(1);
    __syncthreads();

    auto unit = [&](int u, const u32x4 (&wc)[NT], const uint32_t (&sv)[NT]) {
        const int buf = u & 1;
        // the unit k_gemm_lx begins a new partial sum at: fold the running one
        if ((cuts >> (u - cbase)) & 1u) {
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    if (started)
#pragma unroll
                        for (int e = 0; e < 4; e++) tot[mt][nt][e] = tot[mt][nt][e] + seg[mt][nt][e];
                    else
                        tot[mt][nt] = seg[mt][nt];
                    seg[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
                }
            started = true;
        }
        half8_t b[2][NT], bl[2][NT];   // bl: the lo half's fragment, 2^-11 b
        float scale[2][NT];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                b[h][nt] = h ? dequant8_biased(wc[nt][2], wc[nt][3]) : dequant8_biased(wc[nt][0], wc[nt][1]);
                bl[h][nt] = lo_weight8(b[h][nt]);
                scale[h][nt] = rec_scale<F32S>(sv[nt], h);
            }
        // per half-group, every m-tile's MFMA pair first and the scale FMAs
        // after them, so no FMA waits on the MFMA issued just before it; each
        // output's operations and their order are those of k_gemm_lx
#pragma unroll
        for (int h = 0; h < 2; h++) {
            u32x4 xv[MTW][2];
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int q = 0; q < 2; q++) xv[mt][q] = xs[buf][(mw + mt) * 4 + 2 * h + q][lane];
            float4_t pp[MTW][NT];
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    pp[mt][nt] = mfma16x16x32(__builtin_bit_cast(half8_t, xv[mt][0]), b[h][nt], float4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    pp[mt][nt] = mfma16x16x32(__builtin_bit_cast(half8_t, xv[mt][1]), bl[h][nt], pp[mt][nt]);
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int e = 0; e < 4; e++) seg[mt][nt][e] = __builtin_fmaf(scale[h][nt], pp[mt][nt][e], seg[mt][nt][e]);
        }
        if (u + 1 == cend) {   // the plane's value (its last segment folded in) joins the sum
#pragma unroll
            for (int mt = 0; mt < MTW; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    float4_t v = seg[mt][nt];
                    if (started)
#pragma unroll
                        for (int e = 0; e < 4; e++) v[e] = tot[mt][nt][e] + seg[mt][nt][e];
                    if (cp == 0)
                        sum[mt][nt] = v;
                    else
#pragma unroll
                        for (int e = 0; e < 4; e++) sum[mt][nt][e] = sum[mt][nt][e] + v[e];
                    seg[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
                }
            started = false;
            if (cp + 1 < P) {
                cp++;
                cbase = cend;
                cend = lx_plane_start(cp + 1, KU, P);
                cuts = has ? lx_cuts(pair, npairs, Gm, cend - cbase) : 0u;
            }
        }
    };
    int u = 0;
    for (; u + R <= len; u += R) {
#pragma unroll
        for (int I = 0; I < R; I++) {
            load_w(u + I + PW, w[(I + PW) % R], sc[(I + PW) % R]);
            unit(u + I, w[I], sc[I]);
            // the next unit's activations go in the other buffer: every wave
            // finished reading it (one unit ago) before the last barrier
            store_x((I + 1) & 1);
            load_x(u + I + 2);
            __syncthreads();
        }
    }
    // at most PW units remain, their records in ring slots 0 .. PW-1
#pragma unroll
    for (int I = 0; I < PW; I++) {
        if (u + I < len) {
            unit(u + I, w[I], sc[I]);
            store_x((I + 1) & 1);
            load_x(u + I + 2);
            __syncthreads();
        }
    }
    if (!has) return;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int tile = pair * NT + nt;
        if (tile * 16 >= N) continue;
        if (tile * 16 + 16 > N && tile * 16 + (lane & 15) >= N) continue;
#pragma unroll
        for (int mt = 0; mt < MTW; mt++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sum[mt][nt][e]), ro,
                                                      vo + (((mt0 + mw + mt) * 16 + e) * N + tile * 16) * 4, 0, 0);
    }
}

// The planes launch_gemm writes for w at M rows: w.P, or one when the many
// rows give every CU two workgroups or more without the K split
// (k_gemm_tm_sum, 2 <= P < 16).
int gemm_planes(const QTensor& w, int M, int ncu) {
    if (M <= 32 || w.P < 2 || w.P >= 16) return w.P;
    const long long work = (long long)((w.Nt / 2 + TM_PAIRS - 1) / TM_PAIRS) * ((M + 16 * TM_MT - 1) / (16 * TM_MT));
    return work >= 2LL * ncu ? 1 : w.P;
}

template <bool F32S>
static void launch_gemm_fmt(hipStream_t st, const QTensor& w, const uint4* Xp, int xp_mtiles, float* out, int M,
                            int ncu) {
    if (M <= 16) launch_lx<1, F32S>(st, w, Xp, out, M, ncu);
    else if (M <= 32) launch_lx<2, F32S>(st, w, Xp, out, M, ncu);
    else {
        // the same planes and cut points as k_gemm_lx (lx_groups)
        const int Gm = lx_groups(w, ncu) / w.P;
        const int npairs = w.Nt / 2;
        const bool sum = gemm_planes(w, M, ncu) == 1;
        const int nrb = (M + 16 * TM_MT - 1) / (16 * TM_MT);
        // Twelve pairs a workgroup where that takes fewer rounds of
        // workgroups over the CUs, counting a round of the twelve-wave kernel
        // as 1.5 of the eight-wave one's (measured at 128 rows: 39 against
        // 25 us a round at gate|up, 36 against 25 at down): at 128 rows
        // gate|up runs 3 rounds instead of 5 and down 2 instead of 3.
        const int units12 = w.P * ((npairs + TM12_WAVES - 1) / TM12_WAVES);
        const long long r8 = ((long long)w.P * ((npairs + TM_PAIRS - 1) / TM_PAIRS) * nrb + ncu - 1) / ncu;
        const long long r12 = ((long long)units12 * nrb + ncu - 1) / ncu;
        if (!sum && 3 * r12 <= 2 * r8) {
            dim3 grid(8 * ((units12 + 7) / 8) * nrb);
            hipLaunchKernelGGL(k_gemm_tm12<F32S>, grid, dim3(64 * TM12_WAVES), 0, st, (const uint8_t*)w.codes, Xp,
                               xp_mtiles, out, w.KU, M, w.N, w.Nt, w.P, Gm);
            CHECK_LAUNCH();
            return;
        }
        const int units = (sum ? 1 : w.P) * ((npairs + TM_PAIRS - 1) / TM_PAIRS);
        dim3 grid(8 * ((units + 7) / 8) * nrb);
        if (sum)
            hipLaunchKernelGGL(k_gemm_tm_sum<F32S>, grid, dim3(64 * TM_WAVES), 0, st, (const uint8_t*)w.codes, Xp,
                               xp_mtiles, out, w.KU, M, w.N, w.Nt, w.P, Gm);
        else
            hipLaunchKernelGGL(k_gemm_tm<F32S>, grid, dim3(64 * TM_WAVES), 0, st, (const uint8_t*)w.codes, Xp,
                               xp_mtiles, out, w.KU, M, w.N, w.Nt, w.P, Gm);
    }
    CHECK_LAUNCH();
}

void launch_gemm(hipStream_t st, const QTensor& w, const uint4* Xp, int xp_mtiles, float* out, int M, int ncu) {
    if (w.f32s) launch_gemm_fmt<true>(st, w, Xp, xp_mtiles, out, M, ncu);
    else launch_gemm_fmt<false>(st, w, Xp, xp_mtiles, out, M, ncu);
}

// =========================================================== operand prep ===
// Writes 8 consecutive values of row m (columns 8c .. 8c+7) as the f16 hi/lo
// operand fragments of the GEMM (layout above; lo scaled by 2^11).
__device__ static inline void write_hilo(uint4* Xp, int m, int c, int KU, const float* v) {
    const int g = c >> 2, kb = c & 3;
    const int mt = m >> 4, lane = (m & 15) + 16 * kb;
    half8_t hi, lo;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        _Float16 a, b;
        split_hilo_x(v[j], a, b);
        hi[j] = a;
        lo[j] = b;
    }
    const size_t at = (((size_t)mt * 2 * KU + g) * 2) * 64 + lane;
    Xp[at] = __builtin_bit_cast(uint4, hi);
    Xp[at + 64] = __builtin_bit_cast(uint4, lo);
}

__global__ void k_prep_rows(const float* __restrict__ x, int ldx, int M, int Mpad, int K, int KU,
                            uint4* __restrict__ Xp) {
    const int per = 8 * KU;
    const int total = Mpad * per;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int m = i / per, c = i % per;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int k = 8 * c + j;
            v[j] = (m < M && k < K) ? x[(size_t)m * ldx + k] : 0.0f;
        }
        write_hilo(Xp, m, c, KU, v);
    }
}

void launch_prep_rows(hipStream_t st, const float* x, int ldx, int M, int Mpad, int K, int KU,
                      uint4* Xp) {
    const int total = Mpad * 8 * KU;
    hipLaunchKernelGGL(k_prep_rows, dim3((total + 255) / 256), dim3(256), 0, st, x, ldx, M, Mpad, K, KU, Xp);
    CHECK_LAUNCH();
}

// ========================================================= finish kernels ===
// Residual step and rmsnorm, one workgroup of 1024 threads per row, the row
// held in registers (4 columns a thread per pass, H <= 8192):
//   x = x + the projection's K planes added in order (add_inplace,
//   web/model/kernels.js:1334-1346), optionally round_f16 (:1356-1383, the
//   per-block residual round, model.js:619-624), written back;
//   then, with w: rmsnorm (:930-976), y = x * (1/sqrt(ss/H + eps)) * w, as the
//   next matmul's f16 hi/lo operand Xp (or as rows y). ss is summed per wave
//   (butterfly) and then over the waves in order.
// part == nullptr: the x rows as they are, gathered through `rows` (the entry
// rows, the head's sampled rows). Rows M .. Mpad-1 get zero operand rows.
constexpr int RN_THREADS = 1024, RN_PASSES = 2, RN_SPLITS = 16;
__global__ __launch_bounds__(RN_THREADS) void k_resid_norm(float* __restrict__ x, const int32_t* __restrict__ rows,
                                                           const float* __restrict__ part, int splits, int M, int H,
                                                           int round, const float* __restrict__ w, float eps, int KU,
                                                           uint4* __restrict__ Xp, float* __restrict__ y) {
    __shared__ float red[RN_THREADS / 64];
    __shared__ float scale_s;
    const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const int n4 = H >> 2;
    if (m >= M) {
        const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int c8 = t; c8 < 8 * KU; c8 += RN_THREADS) write_hilo(Xp, m, c8, KU, z);
        return;
    }
    const size_t xoff = (size_t)(rows ? rows[m] : m) * H;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 v[RN_PASSES], wv[RN_PASSES];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < RN_PASSES; k++) {
        const int c4 = t + k * RN_THREADS;
        v[k] = wv[k] = zero;
        if (c4 >= n4) continue;
        if (w) wv[k] = *(const float4*)(w + 4 * c4);   // in flight with the row's loads
        float4 xv = *(const float4*)(x + xoff + 4 * c4);
        if (part) {
            // every plane's load in flight at once, through a resource sized
            // to the planes: a load past the last one reads zero (no branch),
            // and adding +0 leaves the in-order sum as it is
            const auto rp = __builtin_amdgcn_make_buffer_rsrc((void*)part, 0, splits * M * H * 4, 0x00020000);
            float4 pv[RN_SPLITS];
#pragma unroll
            for (int s = 0; s < RN_SPLITS; s++) {
                const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rp, (m * H + 4 * c4) * 4, s * M * H * 4, 0);
                pv[s] = make_float4(__uint_as_float(q[0]), __uint_as_float(q[1]), __uint_as_float(q[2]),
                                    __uint_as_float(q[3]));
            }
            float4 p = pv[0];
#pragma unroll
            for (int s = 1; s < RN_SPLITS; s++)
                p = make_float4(p.x + pv[s].x, p.y + pv[s].y, p.z + pv[s].z, p.w + pv[s].w);
            for (int s = RN_SPLITS; s < splits; s++) {
                const float4 q = *(const float4*)(part + ((size_t)s * M + m) * H + 4 * c4);
                p = make_float4(p.x + q.x, p.y + q.y, p.z + q.z, p.w + q.w);
            }
            xv = make_float4(xv.x + p.x, xv.y + p.y, xv.z + p.z, xv.w + p.w);
            if (round)
                xv = make_float4(round_f16_value(xv.x), round_f16_value(xv.y), round_f16_value(xv.z),
                                 round_f16_value(xv.w));
            *(float4*)(x + xoff + 4 * c4) = xv;
        }
        v[k] = xv;
        ss = ss + xv.x * xv.x;
        ss = ss + xv.y * xv.y;
        ss = ss + xv.z * xv.z;
        ss = ss + xv.w * xv.w;
    }
    if (!w) return;   // the residual step alone (the pass's last block)
    ss = wave_sum(ss);
    if (lane == 0) red[t >> 6] = ss;
    __syncthreads();
    if (t == 0) {
        float tot = 0.0f;
        for (int i = 0; i < RN_THREADS / 64; i++) tot = tot + red[i];
        scale_s = 1.0f / sqrtf(tot / (float)H + eps);
    }
    __syncthreads();
    const float scale = scale_s;
#pragma unroll
    for (int k = 0; k < RN_PASSES; k++) {
        const int c4 = t + k * RN_THREADS;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
        if (c4 < n4) {
            o[0] = v[k].x * scale * wv[k].x;
            o[1] = v[k].y * scale * wv[k].y;
            o[2] = v[k].z * scale * wv[k].z;
            o[3] = v[k].w * scale * wv[k].w;
            if (y) *(float4*)(y + (size_t)m * H + 4 * c4) = make_float4(o[0], o[1], o[2], o[3]);
        }
        if (Xp) {
            // lanes (2i, 2i+1) hold the two halves of one 8-column operand chunk
            float e[8];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                e[q] = o[q];
                e[4 + q] = __shfl_xor(o[q], 1);
            }
            if (c4 < n4 && (c4 & 1) == 0) write_hilo(Xp, m, c4 >> 1, KU, e);
        }
    }
    if (Xp) {
        // operand columns past H (K padded to whole 64-column units)
        const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int c8 = (H >> 3) + t; c8 < 8 * KU; c8 += RN_THREADS) write_hilo(Xp, m, c8, KU, z);
    }
}

void launch_resid_norm(hipStream_t st, float* x, const int32_t* rows, const float* part, int splits, int M, int Mpad,
                       int H, int round, const float* w, float eps, int KU, uint4* Xp, float* y) {
    hipLaunchKernelGGL(k_resid_norm, dim3(Xp ? Mpad : M), dim3(RN_THREADS), 0, st, x, rows, part, splits, M, H, round,
                       w, eps, KU, Xp, y);
    CHECK_LAUNCH();
}

// rmsnorm (web/model/kernels.js:930-976) is y = x * f * w with the row factor
// f = 1/sqrt(ss/H + eps); the matmul that follows is linear in its operand,
// so (x*f*w) . W^T = f * ((x*w) . W^T). The residual kernel below writes the
// operand x*w and the row's partial sums of squares; the matmul's consumer
// multiplies the summed planes by f (row_scale). This takes the row-wide
// reduction off the path between the residual step and the matmul, so the
// residual step spreads over (slice, row) workgroups instead of one per row.
// In two parts, so a caller can issue the loads beside its own:
// row_scale_load puts all RW_SMAX loads of row m in flight at once (the
// resource's base is the array's, uniform for any m; the slots past the nsl
// partials read as zero), row_scale_of adds them in order.
struct RowSS {
    float q[RW_SMAX];
};
__device__ static inline RowSS row_scale_load(const RowScale& rs, int m) {
    RowSS r;
    if (!rs.ssp) return r;
    const auto rq = __builtin_amdgcn_make_buffer_rsrc((void*)rs.ssp, 0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int s = 0; s < RW_SMAX; s++) {
        const float v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rq, (m * RW_SMAX + s) * 4, 0, 0));
        r.q[s] = s < rs.nsl ? v : 0.0f;
    }
    return r;
}
__device__ static inline float row_scale_of(const RowScale& rs, const RowSS& r) {
    if (!rs.ssp) return 1.0f;
    float tot = 0.0f;
#pragma unroll
    for (int s = 0; s < RW_SMAX; s++) tot = tot + r.q[s];
    return 1.0f / sqrtf(tot / (float)rs.H + rs.eps);
}
__device__ static inline float row_scale(const RowScale& rs, int m) { return row_scale_of(rs, row_scale_load(rs, m)); }

// Residual step (add_inplace, web/model/kernels.js:1334-1346: x plus the
// projection's planes added in order; optional round_f16, :1356-1383, the
// per-block round of model.js:619-624), then, with w, the next matmul's
// operand x*w as f16 hi/lo and this slice's sum of squares of x (each
// thread's 4 values in order, a wave butterfly, the two waves in order) at
// ssp[m*RW_SMAX + slice]. Workgroup (slice, row): 128 threads, a float4 of
// the row each. part == nullptr: x as it is. Rows M .. Mpad-1 get zero
// operand rows. H % 64 == 0, so the operand has no padding columns. SP plane
// loads are issued at once (4 when the projection has at most 4 planes, so
// no load goes out past them; 16 otherwise), the rest in a loop.
template <int SP>
__global__ __launch_bounds__(RW_THREADS) void k_resid_w(float* __restrict__ x, const float* __restrict__ part,
                                                      int splits, int M, int H, int round,
                                                      const float* __restrict__ w, int KU, uint4* __restrict__ Xp,
                                                      float* __restrict__ ssp) {
    __shared__ float red[RW_THREADS / 64];
    const int m = blockIdx.y, sl = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const int n4 = H >> 2, c4 = sl * RW_THREADS + t;
    const bool live = c4 < n4;
    if (m >= M) {
        if (Xp && live && (c4 & 1) == 0) {
            const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            write_hilo(Xp, m, c4 >> 1, KU, z);
        }
        return;
    }
    const size_t xoff = (size_t)m * H + 4 * (size_t)c4;
    float4 xv = make_float4(0.f, 0.f, 0.f, 0.f), wv = xv;
    if (live) {
        if (w) wv = *(const float4*)(w + 4 * c4);
        xv = *(const float4*)(x + xoff);
        if (part) {
            // every plane's load in flight at once, through a resource sized
            // to the planes: a load past the last one reads zero (no branch),
            // and adding +0 leaves the in-order sum as it is
            const auto rp = __builtin_amdgcn_make_buffer_rsrc((void*)part, 0, splits * M * H * 4, 0x00020000);
            float4 pv[SP];
#pragma unroll
            for (int s = 0; s < SP; s++) {
                const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rp, (int)xoff * 4, s * M * H * 4, 0);
                pv[s] = make_float4(__uint_as_float(q[0]), __uint_as_float(q[1]), __uint_as_float(q[2]),
                                    __uint_as_float(q[3]));
            }
            float4 pp = pv[0];
#pragma unroll
            for (int s = 1; s < SP; s++)
                pp = make_float4(pp.x + pv[s].x, pp.y + pv[s].y, pp.z + pv[s].z, pp.w + pv[s].w);
            for (int s = SP; s < splits; s++) {
                const float4 q = *(const float4*)(part + (size_t)s * M * H + xoff);
                pp = make_float4(pp.x + q.x, pp.y + q.y, pp.z + q.z, pp.w + q.w);
            }
            xv = make_float4(xv.x + pp.x, xv.y + pp.y, xv.z + pp.z, xv.w + pp.w);
            if (round)
                xv = make_float4(round_f16_value(xv.x), round_f16_value(xv.y), round_f16_value(xv.z),
                                 round_f16_value(xv.w));
            *(float4*)(x + xoff) = xv;
        }
    }
    if (!w) return;   // the residual step alone (the pass's last block)
    float ss = 0.0f;
    ss = ss + xv.x * xv.x;
    ss = ss + xv.y * xv.y;
    ss = ss + xv.z * xv.z;
    ss = ss + xv.w * xv.w;
    ss = wave_sum(ss);
    if (lane == 0) red[t >> 6] = ss;
    // lanes (2i, 2i+1) hold the two halves of one 8-column operand chunk
    float o[4] = {xv.x * wv.x, xv.y * wv.y, xv.z * wv.z, xv.w * wv.w};
    float e[8];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        e[q] = o[q];
        e[4 + q] = __shfl_xor(o[q], 1);
    }
    if (live && (c4 & 1) == 0) write_hilo(Xp, m, c4 >> 1, KU, e);
    __syncthreads();
    if (t == 0) {
        float tot = 0.0f;
        for (int i = 0; i < RW_THREADS / 64; i++) tot = tot + red[i];
        ssp[(size_t)m * RW_SMAX + sl] = tot;
    }
}

void launch_resid_w(hipStream_t st, float* x, const float* part, int splits, int M, int Mpad, int H, int round,
                    const float* w, int KU, uint4* Xp, float* ssp) {
    const int nsl = (H / 4 + RW_THREADS - 1) / RW_THREADS;
    const dim3 grid(nsl, w ? Mpad : M);
    if (splits <= 4)
        hipLaunchKernelGGL(k_resid_w<4>, grid, dim3(RW_THREADS), 0, st, x, part, splits, M, H, round, w, KU, Xp, ssp);
    else
        hipLaunchKernelGGL(k_resid_w<RN_SPLITS>, grid, dim3(RW_THREADS), 0, st, x, part, splits, M, H, round, w, KU,
                           Xp, ssp);
    CHECK_LAUNCH();
}

// SwiGLU (web/model/kernels.js:1513-1529 silu_mul): act = g * (1/(1+exp(-g)))
// * up over the fused gate|up projection, straight into the down operand.
// SP > 0: at most SP planes, every plane's loads issued at once (through a
// resource sized to the planes, so those past the last read zero and are not
// added), before the row factor's; SP = 0: any plane count, in a loop.
template <int SP>
__global__ __launch_bounds__(256) void k_fin_swiglu(const float* __restrict__ part, int splits, int M, int Mpad,
                                                    int F, int KU, uint4* __restrict__ Xp, RowScale rs) {
    // one thread per (row, 8 columns); the planes are added in order
    const int per = 8 * KU;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= Mpad * per) return;
    const int m = i / per, c = i % per, k0 = 8 * c;
    const size_t N2 = 2 * (size_t)F, plane = (size_t)M * N2;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (m < M && k0 < F) {
        float g[8], u[8];
        const float* row = part + (size_t)m * N2 + k0;
        const bool fast = k0 + 8 <= F && (F & 3) == 0;
        u32x4 q[SP > 0 ? SP : 1][4];
        if constexpr (SP > 0) {
            // issued by every thread (no branch to join): a thread off the fast
            // path reads in-bounds or zero values it does not use
            const auto rp = __builtin_amdgcn_make_buffer_rsrc((void*)part, 0, (uint32_t)(splits * plane * 4),
                                                              0x00020000);
            const int at = (int)(((size_t)m * N2 + k0) * 4);
#pragma unroll
            for (int s = 0; s < SP; s++) {
                const int so = (int)(s * plane * 4);
                q[s][0] = __builtin_amdgcn_raw_buffer_load_b128(rp, at, so, 0);
                q[s][1] = __builtin_amdgcn_raw_buffer_load_b128(rp, at + 16, so, 0);
                q[s][2] = __builtin_amdgcn_raw_buffer_load_b128(rp, at + 4 * F, so, 0);
                q[s][3] = __builtin_amdgcn_raw_buffer_load_b128(rp, at + 4 * F + 16, so, 0);
            }
        }
        // the gate|up operand carried x*w: rmsnorm's row factor goes on below
        // (its loads issued here, after the planes')
        const RowSS rq = row_scale_load(rs, m);
        if (SP > 0 && fast) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                g[j] = __uint_as_float(q[0][j >> 2][j & 3]);
                u[j] = __uint_as_float(q[0][2 + (j >> 2)][j & 3]);
            }
#pragma unroll
            for (int s = 1; s < SP; s++)
                if (s < splits)
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        g[j] = g[j] + __uint_as_float(q[s][j >> 2][j & 3]);
                        u[j] = u[j] + __uint_as_float(q[s][2 + (j >> 2)][j & 3]);
                    }
        } else if (fast) {
            auto ld8 = [&](const float* p, float* x) {
                const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
                x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
            };
            ld8(row, g);
            ld8(row + F, u);
#pragma unroll 4
            for (int s = 1; s < splits; s++) {
                float gs[8], us[8];
                ld8(row + s * plane, gs);
                ld8(row + s * plane + F, us);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    g[j] = g[j] + gs[j];
                    u[j] = u[j] + us[j];
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                g[j] = u[j] = 0.0f;
                if (k0 + j >= F) continue;
                g[j] = row[j];
                u[j] = row[F + j];
                for (int s = 1; s < splits; s++) {
                    g[j] = g[j] + row[s * plane + j];
                    u[j] = u[j] + row[s * plane + F + j];
                }
            }
        }
        const float f = row_scale_of(rs, rq);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            g[j] = g[j] * f;
            u[j] = u[j] * f;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float sc = 1.0f / (1.0f + expf(-g[j]));
            v[j] = k0 + j < F ? g[j] * sc * u[j] : 0.0f;
        }
    }
    write_hilo(Xp, m, c, KU, v);
}

void launch_fin_swiglu(hipStream_t st, const float* part, int splits, int M, int Mpad, int F, int KU,
                       uint4* Xp, const RowScale& rs) {
    const int total = Mpad * 8 * KU;
    const dim3 grid((total + 255) / 256);
    // the buffer resource's offsets are 32-bit
    const bool small = (size_t)splits * M * 2 * (size_t)F * 4 < (1ull << 31);
    if (small && splits <= 1)
        hipLaunchKernelGGL(k_fin_swiglu<1>, grid, dim3(256), 0, st, part, splits, M, Mpad, F, KU, Xp, rs);
    else if (small && splits <= 4)
        hipLaunchKernelGGL(k_fin_swiglu<4>, grid, dim3(256), 0, st, part, splits, M, Mpad, F, KU, Xp, rs);
    else
        hipLaunchKernelGGL(k_fin_swiglu<0>, grid, dim3(256), 0, st, part, splits, M, Mpad, F, KU, Xp, rs);
    CHECK_LAUNCH();
}

// ============================================================ KV geometry ===
// One (page, kv head) block of the pool, blk = 64*D + 64*ng*4 bytes:
//   K: codes [64 tokens][D] with column d at (D/4)*((d%32)/8) + 8*(d/32) + d%8,
//      so one lane's fragment bytes for every group are contiguous; then f32
//      scales [64 tokens][ng].
//   V: codes [4][D][16]: with v = vpos(s) = 16*((s%16)/4) + 4*(s/16) + s%4,
//      token s's code for channel d sits in 16-byte row (v/16, d) at byte
//      v%16, so a lane's P·V fragment (16 tokens of one channel) is one
//      contiguous 16-byte load, and one token's D codes lie in D*16 bytes
//      (a new token dirties 16 lines of 128 B at D = 128, not the 64 of a
//      [D][64] layout); then f32 scales [4][ng][16] at the same positions.
// Codes are stored biased (code ^ 0x80, i.e. code + 128) so the MFMA dequant
// puts them under an f16 exponent directly; they are the reference's store_kv
// codes bit for bit once converted back (k_kv_ref: cc_read_kv, cc_write_kv).
__host__ __device__ static inline int kpos(int d, int D) { return (D / 4) * ((d & 31) >> 3) + 8 * (d >> 5) + (d & 7); }
__host__ __device__ static inline int vpos(int s) { return 16 * ((s & 15) >> 2) + 4 * (s >> 4) + (s & 3); }
// byte of V code (channel d, token s) in its block, and float of V scale
// (group b, token s) after the codes
__host__ __device__ static inline int vcode_at(int d, int s, int D) {
    const int v = vpos(s);
    return ((v >> 4) * D + d) * 16 + (v & 15);
}
__host__ __device__ static inline int vscale_at(int b, int s, int ng) {
    const int v = vpos(s);
    return ((v >> 4) * ng + b) * 16 + (v & 15);
}

// store_kv (web/model/kernels.js:1024-1073) for a row's K and V, plus RoPE on
// its Q (kernels.js:1093-1129) into the attention operand, after the q|k|v
// splits are summed.
// Bit-exact with the reference given the same q|k|v row: RoPE a*cs - o*sn
// (no fused multiply-add: the build passes -ffp-contract=off), amax,
// scale = amax/127, inv = scale > 0 ? 1/scale : 0, rint, clamp ±127.
// Channel c of one head after split-half RoPE, given the (cos, sin) of c's
// pair at the row's position (tbl[(pos*(rot/2) + c mod rot/2)*2 + 0/1]);
// channels from rot on pass through.
__device__ static inline float rope_cs(const float* src, int c, int rot, float cs, float sn) {
    if (c >= rot) return src[c];
    const int half = rot >> 1;
    if (c < half) {
        const float a = src[c], o = src[c + half];
        return a * cs - o * sn;
    }
    const float a = src[c - half], o = src[c];
    return o * cs + a * sn;
}

// Spread over (row, head): one wave per head of a row, four heads per
// workgroup. The head's D values (K splits summed in order) sit in the wave's
// LDS slice; Q heads are RoPE'd into the attention operand, K heads RoPE'd and
// quantised into the pool, V heads quantised.
template <int D, int SU>
__global__ __launch_bounds__(256) void k_fin_qkv(const float* __restrict__ part, int splits, int M,
                                                  const int32_t* __restrict__ row_job,
                                                  const JobDev* __restrict__ jobs, int nH, int group, KVGeom g,
                                                  const float* __restrict__ tbl, int rot, uint8_t* __restrict__ kpool,
                                                  uint8_t* __restrict__ vpool,
                                                  const uint32_t* __restrict__ page_table, uint4* __restrict__ Qp,
                                                  RowScale rs, int do_q, int do_kv, QkExtras ex) {
    __shared__ float buf[4][D];
    __shared__ __attribute__((aligned(16))) float rq[4][D];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m = blockIdx.y;
    const int nKV = g.nKV;
    const int nqkv = nH + 2 * nKV;
    const int nall = nqkv + (ex.gate ? nH : 0);   // a hybrid block's gate heads follow v
    const int hidx = blockIdx.x * 4 + wave;
    const bool live = hidx < nall;
    const int N = nall * D;
    // SU planes' loads in flight at once, first (4 when q|k|v has at most 4
    // planes, else 16), through a resource sized to the planes: past the last
    // one a load reads zero (no branch), and adding +0 leaves the in-order sum
    // as it is; planes past SU in a loop
    constexpr int DH = D / 64;
    float pv[DH][SU];
    if (live) {
        const auto rp = __builtin_amdgcn_make_buffer_rsrc((void*)part, 0, splits * M * N * 4, 0x00020000);
#pragma unroll
        for (int h = 0; h < DH; h++) {
            const int at = (m * N + hidx * D + 64 * h + lane) * 4;
#pragma unroll
            for (int s = 0; s < SU; s++)
                pv[h][s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, at, s * M * N * 4, 0));
        }
    }
    // the row's job and its page, and rmsnorm's row factor (the q|k|v operand
    // carried x*w), looked up while the planes load
    const JobDev jb = jobs[row_job[m]];
    const int i = m - jb.row0;
    const int pos = jb.past + i;
    const uint32_t page = page_table[(size_t)jb.slot * g.max_pages + pos / g.page];
    const float f = row_scale(rs, m);
    // RoPE's (cos, sin) for this lane's channels 64h + lane at pos, loaded
    // here so they are in flight beside the planes
    float cs[DH], sn[DH];
    {
        const int half = rot >> 1;
#pragma unroll
        for (int h = 0; h < DH; h++) {
            const int c = 64 * h + lane;
            cs[h] = 1.0f;
            sn[h] = 0.0f;
            if (c < rot) {
                const float2 t2 = *(const float2*)(tbl + ((size_t)pos * half + (c < half ? c : c - half)) * 2);
                cs[h] = t2.x;
                sn[h] = t2.y;
            }
        }
    }
    if (live) {
#pragma unroll
        for (int h = 0; h < DH; h++) {
            float p = pv[h][0];
#pragma unroll
            for (int s = 1; s < SU; s++) p = p + pv[h][s];
            for (int s = SU; s < splits; s++) p = p + part[((size_t)s * M + m) * N + hidx * D + 64 * h + lane];
            buf[wave][64 * h + lane] = p * f;
        }
    }
    __syncthreads();
    // q_norm / k_norm (model.js:388-394): rmsnorm over the head's D values
    // (lane partials, then a wave reduction), before RoPE reads neighbouring
    // channels
    if (ex.qn) {   // a kernel argument: the barrier is uniform
        if (live && hidx < nH + nKV) {
            const float* w = hidx < nH ? ex.qn : ex.kn;
            float ss = 0.0f;
            for (int d = lane; d < D; d += 64) ss += buf[wave][d] * buf[wave][d];
            ss = wave_sum(ss);
            const float scale = 1.0f / sqrtf(ss / (float)D + ex.eps);
            for (int d = lane; d < D; d += 64) buf[wave][d] = buf[wave][d] * scale * w[d];
        }
        __syncthreads();
    }
    if (live && hidx < nH) {
        if (do_q) {
#pragma unroll
            for (int h = 0; h < DH; h++) rq[wave][64 * h + lane] = rope_cs(buf[wave], 64 * h + lane, rot, cs[h], sn[h]);
        }
    }
    __syncthreads();
    if (!live) return;
    if (hidx >= nqkv) {
        // the output gate's raw values (times the row factor), for the combine
        if (do_q) {
            float* gr = ex.gate + (size_t)m * nH * D + (size_t)(hidx - nqkv) * D;
            for (int d = lane; d < D; d += 64) gr[d] = buf[wave][d];
        }
        return;
    }
    if (hidx < nH) {
        if (!do_q) return;
        if (lane < D / 8) {
            const int d0 = 8 * lane;
            half8_t hi, lo;
            // the lane's 8 channels as two 16-byte reads
            const float4 qa = *(const float4*)&rq[wave][d0], qb = *(const float4*)&rq[wave][d0 + 4];
            const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                _Float16 a, b;
                split_hilo(qv[j], a, b);
                hi[j] = a;
                lo[j] = b;
            }
            const int kvh = hidx / group, gi = hidx % group;
            const int rho = i * group + gi;
            const int mtq = rho >> 4, ln = (rho & 15) + 16 * ((d0 & 31) >> 3), grp = d0 >> 5;
            const size_t at = (size_t)jb.qp_off + ((((size_t)kvh * jb.mtq + mtq) * g.ng + grp) * 2) * 64 + ln;
            Qp[at] = __builtin_bit_cast(uint4, hi);
            Qp[at + 64] = __builtin_bit_cast(uint4, lo);
        }
        return;
    }
    if (!do_kv) return;
    const int which = hidx < nH + nKV ? 0 : 1;
    const int n = hidx - nH - which * nKV;
    const int s = pos % g.page;
    uint8_t* blk = (which ? vpool : kpool) + ((size_t)page * nKV + n) * g.blk;
#pragma unroll
    for (int h = 0; h < DH; h++) {
        const int d = 64 * h + lane;
        const float v = which ? buf[wave][d] : rope_cs(buf[wave], d, rot, cs[h], sn[h]);
        float amax = fabsf(v);
        for (int o = 1; o < 32; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
        const float scale = amax / 127.0f;
        const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        float q = __builtin_rintf(v * inv);
        q = fminf(fmaxf(q, -127.0f), 127.0f);
        const int8_t code = (int8_t)(int)q;
        const int b = d >> 5;
        if (which == 0) {
            blk[(size_t)s * D + kpos(d, D)] = (uint8_t)((uint8_t)code ^ 0x80u);
            if ((d & 31) == 0) *(float*)(blk + 64 * D + ((size_t)s * g.ng + b) * 4) = scale;
        } else {
            blk[vcode_at(d, s, D)] = (uint8_t)((uint8_t)code ^ 0x80u);
            if ((d & 31) == 0) *(float*)(blk + 64 * D + (size_t)vscale_at(b, s, g.ng) * 4) = scale;
        }
    }
}

template <int D>
static void launch_fin_qkv_d(hipStream_t st, dim3 grid, const float* part, int splits, int M, const int32_t* row_job,
                             const JobDev* jobs, int nH, int group, const KVGeom& g, const float* tbl, int rot,
                             uint8_t* kpool, uint8_t* vpool, const uint32_t* page_table, uint4* Qp,
                             const RowScale& rs, int do_q, int do_kv, const QkExtras& ex) {
    if (splits <= 4)
        hipLaunchKernelGGL((k_fin_qkv<D, 4>), grid, dim3(256), 0, st, part, splits, M, row_job, jobs, nH, group, g,
                           tbl, rot, kpool, vpool, page_table, Qp, rs, do_q, do_kv, ex);
    else
        hipLaunchKernelGGL((k_fin_qkv<D, 16>), grid, dim3(256), 0, st, part, splits, M, row_job, jobs, nH, group, g,
                           tbl, rot, kpool, vpool, page_table, Qp, rs, do_q, do_kv, ex);
}

void launch_fin_qkv(hipStream_t st, const float* part, int splits, int M, const int32_t* row_job,
                    const JobDev* jobs, int nH, int group, const KVGeom& g, const float* tbl, int rot,
                    uint8_t* kpool, uint8_t* vpool, const uint32_t* page_table, uint4* Qp, const RowScale& rs,
                    int do_q, int do_kv, const QkExtras& ex) {
    const int nall = nH + 2 * g.nKV + (ex.gate ? nH : 0);
    const dim3 grid((nall + 3) / 4, M);
    if (g.D == 256)
        launch_fin_qkv_d<256>(st, grid, part, splits, M, row_job, jobs, nH, group, g, tbl, rot, kpool, vpool,
                              page_table, Qp, rs, do_q, do_kv, ex);
    else if (g.D == 128)
        launch_fin_qkv_d<128>(st, grid, part, splits, M, row_job, jobs, nH, group, g, tbl, rot, kpool, vpool,
                              page_table, Qp, rs, do_q, do_kv, ex);
    else
        launch_fin_qkv_d<64>(st, grid, part, splits, M, row_job, jobs, nH, group, g, tbl, rot, kpool, vpool,
                             page_table, Qp, rs, do_q, do_kv, ex);
    CHECK_LAUNCH();
}

// =========================================================== Gated DeltaNet ===
// A hybrid checkpoint's linear_attention blocks (web/model/model.js:418-527,
// web/model/kernels.js:1531-1839) over the packed jobs, each on its own
// session's state. Three kernels after the fused in_proj matmul:
//   k_lin_conv  planes summed (times the input rmsnorm's row factor), the
//               depthwise causal conv + SiLU through the job's rows with the
//               session's ring, the ring advanced; z, b, a passed through;
//   k_gdn       the gated delta rule with the q/k l2norm folded in;
//   k_lin_norm  RMSNormGated times silu(z) into the out_proj operand.

// Plane sum of one column in plane order, times the row factor.
__device__ static inline float plane_col(const float* part, int splits, int M, int N, int m, int col, float f) {
    float p = part[(size_t)m * N + col];
    for (int s = 1; s < splits; s++) p = p + part[((size_t)s * M + m) * N + col];
    return p * f;
}

// causal_conv1d (kernels.js:1538-1580) + update_conv_history (:1582-1620).
// One thread per (job, channel) walks the job's rows in order, so the ring
// (the K-1 raw rows before the current one) stays in registers: it is read
// from the session's state first (zeros for a job at position 0, a new
// session) and written back after the job's last row. Per row: acc = sum over
// k of w[c][k] * x[t-(K-1)+k] in k order, out = acc * (1/(1+exp(-acc))).
// Speculation (model.js:447-470): a rollback job starts from the snapshot's
// ring, advances it through the kept rows' stored raw values and copies
// their stored outputs (and b, a) to `lrep` for the recurrence; a verify
// writes the ring it starts from to the snapshot and stores each row's raw
// value and output. The thread that reads a stored row is the one that
// overwrites it, so a rollback job that is also a verify is ordered.
__global__ __launch_bounds__(256) void k_lin_conv(const float* __restrict__ part, int splits, int M,
                                                  const JobDev* __restrict__ jobs, RowScale rs,
                                                  const float* __restrict__ conv, LinGeom lg,
                                                  float* __restrict__ state, float* __restrict__ lraw,
                                                  float* __restrict__ lrep) {
    constexpr int K = LIN_CONV_K;
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= lg.W) return;
    const int j = blockIdx.y;
    const JobDev jb = jobs[j];
    float* base = state + (size_t)jb.slot * lg.sstride;
    float* rep = base + lg.rep_off;
    float* lr = lrep + (size_t)j * LIN_SPEC_ROWS * lg.lrep_w;
    const int keep = jb.keep > 0 ? jb.keep : 0;
    // plane column: q|k|v|z in place, b and a each padded to nVp rows
    const int col = c < lg.convDim + lg.valueDim + lg.nV ? c : c - lg.nV + lg.nVp;
    if (c >= lg.convDim) {
        // z, b, a pass through; b and a also feed a rollback's and a verify's rows
        const bool ba = c >= lg.convDim + lg.valueDim;
        const int e = c - lg.convDim - lg.valueDim;   // b: [0, nV), a: [nV, 2nV)
        if (ba)
            for (int i = 0; i < keep; i++)
                lr[(size_t)i * lg.lrep_w + lg.convDim + e] = rep[(size_t)i * lg.rep_w + 2 * lg.convDim + e];
        for (int i = 0; i < jb.n; i++) {
            const int m = jb.row0 + i;
            const float v = plane_col(part, splits, M, lg.N, m, col, row_scale(rs, m));
            lraw[(size_t)m * lg.W + c] = v;
            if (ba && jb.snap) rep[(size_t)i * lg.rep_w + 2 * lg.convDim + e] = v;
        }
        return;
    }
    float* cur = base + lg.hist_off + c;            // [K-1][convDim]
    float* snap = base + lg.blk + lg.hist_off + c;
    const float* src = jb.keep >= 0 ? snap : cur;
    float h[K - 1];
#pragma unroll
    for (int r = 0; r < K - 1; r++) h[r] = jb.past > 0 ? src[(size_t)r * lg.convDim] : 0.0f;
    for (int i = 0; i < keep; i++) {
        lr[(size_t)i * lg.lrep_w + c] = rep[(size_t)i * lg.rep_w + lg.convDim + c];
#pragma unroll
        for (int k = 0; k < K - 2; k++) h[k] = h[k + 1];
        h[K - 2] = rep[(size_t)i * lg.rep_w + c];
    }
    if (jb.snap) {
#pragma unroll
        for (int r = 0; r < K - 1; r++) snap[(size_t)r * lg.convDim] = h[r];
    }
    float w[K];
#pragma unroll
    for (int k = 0; k < K; k++) w[k] = conv[(size_t)c * K + k];
    for (int i = 0; i < jb.n; i++) {
        const int m = jb.row0 + i;
        const float x = plane_col(part, splits, M, lg.N, m, col, row_scale(rs, m));
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < K - 1; k++) acc = acc + w[k] * h[k];
        acc = acc + w[K - 1] * x;
        const float sg = 1.0f / (1.0f + expf(-acc));
        const float out = acc * sg;
        lraw[(size_t)m * lg.W + c] = out;
        if (jb.snap) {
            rep[(size_t)i * lg.rep_w + c] = x;
            rep[(size_t)i * lg.rep_w + lg.convDim + c] = out;
        }
#pragma unroll
        for (int k = 0; k < K - 2; k++) h[k] = h[k + 1];
        h[K - 2] = x;
    }
#pragma unroll
    for (int r = 0; r < K - 1; r++) cur[(size_t)r * lg.convDim] = h[r];
}

void launch_lin_conv(hipStream_t st, const float* part, int splits, int M, int njobs, const JobDev* jobs,
                     const RowScale& rs, const float* conv, const LinGeom& lg, float* state, float* lraw,
                     float* lrep) {
    if (njobs <= 0) return;
    hipLaunchKernelGGL(k_lin_conv, dim3((lg.W + 255) / 256, njobs), dim3(256), 0, st, part, splits, M, jobs, rs,
                       conv, lg, state, lraw, lrep);
    CHECK_LAUNCH();
}

// The same conv for a pass with a long job (a prefill chunk), parallel over
// rows, in three steps (the arithmetic per row is the one above, so the bits
// do not depend on the path):
//   k_lin_ring_pre   the ring each job starts from (the session's, or the
//                    snapshot's advanced through the kept rows) into `lring`
//                    [job][K-1][convDim]; the rollback rows to `lrep`; a
//                    verify's snapshot ring;
//   k_lin_conv_rows  one thread per (row, channel): the window from the
//                    job's own rows (planes summed again) and `lring`;
//   k_lin_ring_post  the ring after the job's last row, into the session.
__global__ __launch_bounds__(256) void k_lin_ring_pre(const JobDev* __restrict__ jobs, LinGeom lg,
                                                      float* __restrict__ state, float* __restrict__ lrep,
                                                      float* __restrict__ lring) {
    constexpr int K = LIN_CONV_K;
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= lg.W) return;
    const int j = blockIdx.y;
    const JobDev jb = jobs[j];
    float* base = state + (size_t)jb.slot * lg.sstride;
    const float* rep = base + lg.rep_off;
    float* lr = lrep + (size_t)j * LIN_SPEC_ROWS * lg.lrep_w;
    const int keep = jb.keep > 0 ? jb.keep : 0;
    if (c >= lg.convDim) {
        if (c >= lg.convDim + lg.valueDim) {
            const int e = c - lg.convDim - lg.valueDim;
            for (int i = 0; i < keep; i++)
                lr[(size_t)i * lg.lrep_w + lg.convDim + e] = rep[(size_t)i * lg.rep_w + 2 * lg.convDim + e];
        }
        return;
    }
    float* cur = base + lg.hist_off + c;
    float* snap = base + lg.blk + lg.hist_off + c;
    const float* src = jb.keep >= 0 ? snap : cur;
    float h[K - 1];
#pragma unroll
    for (int r = 0; r < K - 1; r++) h[r] = jb.past > 0 ? src[(size_t)r * lg.convDim] : 0.0f;
    for (int i = 0; i < keep; i++) {
        lr[(size_t)i * lg.lrep_w + c] = rep[(size_t)i * lg.rep_w + lg.convDim + c];
#pragma unroll
        for (int k = 0; k < K - 2; k++) h[k] = h[k + 1];
        h[K - 2] = rep[(size_t)i * lg.rep_w + c];
    }
    float* e = lring + (size_t)j * (K - 1) * lg.convDim + c;
#pragma unroll
    for (int r = 0; r < K - 1; r++) {
        e[(size_t)r * lg.convDim] = h[r];
        if (jb.snap) snap[(size_t)r * lg.convDim] = h[r];
    }
}

__global__ __launch_bounds__(256) void k_lin_conv_rows(const float* __restrict__ part, int splits, int M,
                                                       const int32_t* __restrict__ row_job,
                                                       const JobDev* __restrict__ jobs, RowScale rs,
                                                       const float* __restrict__ conv, LinGeom lg,
                                                       float* __restrict__ state, const float* __restrict__ lring,
                                                       float* __restrict__ lraw) {
    constexpr int K = LIN_CONV_K;
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int m = blockIdx.y;
    if (c >= lg.W || m >= M) return;
    const int j = row_job[m];
    const JobDev jb = jobs[j];
    const int i = m - jb.row0;
    float* rep = state + (size_t)jb.slot * lg.sstride + lg.rep_off;
    const int col = c < lg.convDim + lg.valueDim + lg.nV ? c : c - lg.nV + lg.nVp;
    if (c >= lg.convDim) {
        const float v = plane_col(part, splits, M, lg.N, m, col, row_scale(rs, m));
        lraw[(size_t)m * lg.W + c] = v;
        if (jb.snap && c >= lg.convDim + lg.valueDim) rep[(size_t)i * lg.rep_w + 2 * lg.convDim + (c - lg.convDim - lg.valueDim)] = v;
        return;
    }
    const float* e = lring + (size_t)j * (K - 1) * lg.convDim + c;
    float x[K];   // the window: rows i-K+1 .. i
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int t = i - (K - 1) + k;
        x[k] = t >= 0 ? plane_col(part, splits, M, lg.N, jb.row0 + t, col, row_scale(rs, jb.row0 + t))
                      : e[(size_t)(K - 1 + t) * lg.convDim];
    }
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < K; k++) acc = acc + conv[(size_t)c * K + k] * x[k];
    const float sg = 1.0f / (1.0f + expf(-acc));
    const float out = acc * sg;
    lraw[(size_t)m * lg.W + c] = out;
    if (jb.snap) {
        rep[(size_t)i * lg.rep_w + c] = x[K - 1];
        rep[(size_t)i * lg.rep_w + lg.convDim + c] = out;
    }
}

__global__ __launch_bounds__(256) void k_lin_ring_post(const float* __restrict__ part, int splits, int M,
                                                       const JobDev* __restrict__ jobs, RowScale rs, LinGeom lg,
                                                       float* __restrict__ state, const float* __restrict__ lring) {
    constexpr int K = LIN_CONV_K;
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= lg.convDim) return;
    const int j = blockIdx.y;
    const JobDev jb = jobs[j];
    float* cur = state + (size_t)jb.slot * lg.sstride + lg.hist_off + c;
    const float* e = lring + (size_t)j * (K - 1) * lg.convDim + c;
#pragma unroll
    for (int r = 0; r < K - 1; r++) {
        const int t = jb.n - (K - 1) + r;   // the ring's row r after the job
        cur[(size_t)r * lg.convDim] = t >= 0 ? plane_col(part, splits, M, lg.N, jb.row0 + t, c, row_scale(rs, jb.row0 + t))
                                             : e[(size_t)(K - 1 + t) * lg.convDim];
    }
}

void launch_lin_conv_rows(hipStream_t st, const float* part, int splits, int M, int njobs, const int32_t* row_job,
                          const JobDev* jobs, const RowScale& rs, const float* conv, const LinGeom& lg, float* state,
                          float* lraw, float* lrep, float* lring) {
    if (njobs <= 0 || M <= 0) return;
    const int bw = (lg.W + 255) / 256;
    hipLaunchKernelGGL(k_lin_ring_pre, dim3(bw, njobs), dim3(256), 0, st, jobs, lg, state, lrep, lring);
    hipLaunchKernelGGL(k_lin_conv_rows, dim3(bw, M), dim3(256), 0, st, part, splits, M, row_job, jobs, rs, conv, lg,
                       state, lring, lraw);
    hipLaunchKernelGGL(k_lin_ring_post, dim3((lg.convDim + 255) / 256, njobs), dim3(256), 0, st, part, splits, M, jobs,
                       rs, lg, state, lring);
    CHECK_LAUNCH();
}

// gated_delta_net_step (kernels.js:1672-1805) for every row of a job, on its
// session's S [nV][Dk][Dv]: one workgroup per (value-column tile, value head,
// job), GDN_KS k-groups x GDN_TV columns; each thread holds DK/GDN_KS rows of
// its column for the whole job. Per token, in the reference's arithmetic:
//   g = exp(-exp(A_log) * softplus(a + dt_bias)), beta = sigmoid(b);
//   s *= g; kv = s.k, qo = s.q over k; kq = k.q;
//   delta = (v - kv) * beta; s += k * delta; out = (qo + delta*kq) / sqrt(Dk).
// l2norm_heads (kernels.js:1622-1670) of the head's q and k (source head
// h / group, the value-head repeat) is folded in: the raw dot products and
// the sums of squares share the token's one reduction through LDS (double
// buffered on token parity, one barrier a token), and the factors
// 1/sqrt(sum x^2 + 1e-6) are applied after it; the state update uses the
// normalised k. A job at position 0 starts from a zero state. A rollback
// job starts from the snapshot and first re-runs the kept rows (from `lrep`,
// no output); a verify writes the state it starts from to the snapshot.
constexpr int GDN_KS = 8, GDN_TV = 32;
template <int DK>
__global__ __launch_bounds__(GDN_KS * GDN_TV) void k_gdn(const float* __restrict__ lraw, const float* __restrict__ lrep,
                                                         const JobDev* __restrict__ jobs,
                                                         const float* __restrict__ gp, LinGeom lg,
                                                         float* __restrict__ state, float* __restrict__ core) {
    constexpr int ROWS = DK / GDN_KS;
    __shared__ float pkv[2][GDN_KS][GDN_TV];
    __shared__ float pqo[2][GDN_KS][GDN_TV];
    __shared__ float psc[2][GDN_KS][3];   // k.q, q.q, k.k per k-group
    const int h = blockIdx.y;
    const int j = blockIdx.z;
    const JobDev jb = jobs[j];
    const int col = threadIdx.x % GDN_TV, kg = threadIdx.x / GDN_TV;
    const int vv = blockIdx.x * GDN_TV + col;
    const bool live = vv < lg.Dv;
    const int vvc = live ? vv : lg.Dv - 1;   // out-of-range columns read a real one and discard it
    const int k0 = kg * ROWS;
    const int kh = h / lg.group;
    float* base = state + (size_t)jb.slot * lg.sstride + (size_t)h * DK * lg.Dv;
    float* S = base;                // current
    float* Ssnap = base + lg.blk;   // snapshot
    const float* src = jb.keep >= 0 ? Ssnap : S;
    float s[ROWS];
#pragma unroll
    for (int i = 0; i < ROWS; i++) s[i] = (jb.past > 0 && live) ? src[(size_t)(k0 + i) * lg.Dv + vv] : 0.0f;
    const float A = expf(gp[h]), dtb = gp[lg.nV + h];
    const float q_scale = 1.0f / sqrtf((float)DK);
    int t = 0;   // tokens so far: the LDS buffers alternate on its parity
    // One token: q, k, v at their channel offsets in `row`, b and a at
    // boff + h and boff + nV + h. Every thread reaches its one barrier.
    auto token = [&](const float* row, int boff, float* out) {
        const float* qr = row + kh * DK;
        const float* kr = row + lg.keyDim + kh * DK;
        const float a = row[boff + lg.nV + h] + dtb;
        const float sp = a > 20.0f ? a + logf(1.0f + expf(-a)) : logf(1.0f + expf(a));
        const float g = expf(-A * sp);
        const float beta = 1.0f / (1.0f + expf(-row[boff + h]));
        const int buf = t & 1;
        float kv = 0.0f, qo = 0.0f, kq = 0.0f, qq = 0.0f, kk = 0.0f;
        float kx[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const float ki = kr[k0 + r], qi = qr[k0 + r];
            kx[r] = ki;
            s[r] = s[r] * g;
            kv = kv + s[r] * ki;
            qo = qo + s[r] * qi;
            kq = kq + ki * qi;
            qq = qq + qi * qi;
            kk = kk + ki * ki;
        }
        pkv[buf][kg][col] = kv;
        pqo[buf][kg][col] = qo;
        if (col == 0) {
            psc[buf][kg][0] = kq;
            psc[buf][kg][1] = qq;
            psc[buf][kg][2] = kk;
        }
        __syncthreads();
        float kvT = 0.0f, qoT = 0.0f, kqT = 0.0f, qqT = 0.0f, kkT = 0.0f;
#pragma unroll
        for (int q = 0; q < GDN_KS; q++) {
            kvT = kvT + pkv[buf][q][col];
            qoT = qoT + pqo[buf][q][col];
            kqT = kqT + psc[buf][q][0];
            qqT = qqT + psc[buf][q][1];
            kkT = kkT + psc[buf][q][2];
        }
        const float rq = 1.0f / sqrtf(qqT + 1e-6f), rk = 1.0f / sqrtf(kkT + 1e-6f);
        const float delta = (row[2 * lg.keyDim + h * lg.Dv + vvc] - kvT * rk) * beta;
#pragma unroll
        for (int r = 0; r < ROWS; r++) s[r] = s[r] + (kx[r] * rk) * delta;
        if (out && kg == 0 && live) *out = (qoT * rq + delta * (kqT * rq * rk)) * q_scale;
        t++;
    };
    // a rollback re-runs the kept rows of the session's last verify
    const float* lr = lrep + (size_t)j * LIN_SPEC_ROWS * lg.lrep_w;
    for (int i = 0; i < jb.keep; i++) token(lr + (size_t)i * lg.lrep_w, lg.convDim, nullptr);
    if (jb.snap && live) {
#pragma unroll
        for (int i = 0; i < ROWS; i++) Ssnap[(size_t)(k0 + i) * lg.Dv + vv] = s[i];
    }
    for (int i = 0; i < jb.n; i++) {
        const int m = jb.row0 + i;
        token(lraw + (size_t)m * lg.W, lg.convDim + lg.valueDim, core + (size_t)m * lg.valueDim + h * lg.Dv + vv);
    }
    if (live) {
#pragma unroll
        for (int i = 0; i < ROWS; i++) S[(size_t)(k0 + i) * lg.Dv + vv] = s[i];
    }
}

void launch_gdn(hipStream_t st, const float* lraw, const float* lrep, int njobs, const JobDev* jobs, const float* gp,
                const LinGeom& lg, float* state, float* core) {
    if (njobs <= 0) return;
    const dim3 grid((lg.Dv + GDN_TV - 1) / GDN_TV, lg.nV, njobs), blk(GDN_KS * GDN_TV);
    switch (lg.Dk) {
        case 16: hipLaunchKernelGGL(k_gdn<16>, grid, blk, 0, st, lraw, lrep, jobs, gp, lg, state, core); break;
        case 32: hipLaunchKernelGGL(k_gdn<32>, grid, blk, 0, st, lraw, lrep, jobs, gp, lg, state, core); break;
        case 64: hipLaunchKernelGGL(k_gdn<64>, grid, blk, 0, st, lraw, lrep, jobs, gp, lg, state, core); break;
        default: hipLaunchKernelGGL(k_gdn<128>, grid, blk, 0, st, lraw, lrep, jobs, gp, lg, state, core); break;
    }
    CHECK_LAUNCH();
}

// RMSNormGated (model.js:523-524: rmsnorm over each value head's Dv values
// with gated_norm, then silu_mul(z, normed)) into the out_proj operand. One
// wave per (row, value head), 8 columns a lane.
__global__ __launch_bounds__(256) void k_lin_norm(const float* __restrict__ core, const float* __restrict__ lraw,
                                                  const float* __restrict__ gnorm, float eps, int M, LinGeom lg,
                                                  int KU, uint4* __restrict__ Xp) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = blockIdx.x * 4 + wave, m = blockIdx.y;
    if (h >= lg.nV || m >= M) return;
    const int d0 = 8 * lane;
    const bool act = d0 < lg.Dv;
    float v[8];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        v[j] = act ? core[(size_t)m * lg.valueDim + h * lg.Dv + d0 + j] : 0.0f;
        ss += v[j] * v[j];
    }
    ss = wave_sum(ss);
    if (!act) return;
    const float scale = 1.0f / sqrtf(ss / (float)lg.Dv + eps);
    const float* z = lraw + (size_t)m * lg.W + lg.convDim + h * lg.Dv + d0;
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float y = v[j] * scale * gnorm[d0 + j];
        const float sg = 1.0f / (1.0f + expf(-z[j]));
        o[j] = z[j] * sg * y;
    }
    write_hilo(Xp, m, (h * lg.Dv + d0) >> 3, KU, o);
}

void launch_lin_norm(hipStream_t st, const float* core, const float* lraw, const float* gnorm, float eps, int M,
                     const LinGeom& lg, int KU, uint4* Xp) {
    if (M <= 0) return;
    hipLaunchKernelGGL(k_lin_norm, dim3((lg.nV + 3) / 4, M), dim3(256), 0, st, core, lraw, gnorm, eps, M, lg, KU, Xp);
    CHECK_LAUNCH();
}

// ================================================================ attention ===
// Ragged GQA attention over each chat's own int8 pages
// (web/model/kernels.js:1140-1310 qk_scores_gqa, causal_softmax, attn_av_gqa,
// driven per segment by web/model/model.js:321-351). Every K/V byte of a kv
// head is read once for all the job's query rows rho = i*group + gi of it:
//   S^T[token][rho] = sum_g sk[token][g] * (K_g . Qhi_g + K_g . Qlo_g) on MFMA,
//   masked to token < T_act and token <= past + i (causal inside a verify or
//   prefill run), scaled by 1/sqrt(D);
//   O^T[d][rho] += V^T[d][token] . (p * sv[token][d/32]) (hi/lo) on MFMA.
// The reference's softmax is exact three-pass; this one is online (per page)
// with a log-sum-exp merge of the chunks, equal within tolerance.
// Attention, one wave per work item: (job, kv head, query m-tile, chunk of
// `ppw` pages). The wave walks its pages in order and keeps an online softmax
// (running max, sum, rescaled O) across them; its (max, sum, O) partial for
// the 16 query rows goes to `part` (16 rows of D + 4 floats: max in log2
// units, sum, two pad floats, O). Per page: S^T = K . Q^T (hi/lo)
// scaled per (token, 32-block), masked (token < T_act, token <= past + i) and
// scaled by 1/sqrt(D); O^T += V^T . (p * sv) (hi/lo).
//
// Latency: as soon as S is formed the wave issues the next page's loads — its
// K and V scale blocks (1 KiB each, 16 B a lane into registers, written to
// the wave's LDS slice when that page starts), then its K codes into the K
// registers — and after the PV products the next page's V codes into the V
// registers. So one page of codes is held in registers (two waves per SIMD),
// and no load waits at its point of use. (Loading the scales straight into
// LDS instead makes the compiler wait for those in-flight loads before any
// LDS read it cannot prove apart from them.) Scheduling barriers keep the
// compiler from hoisting the V dequantisation into the S phase, which would
// make S wait for the V loads.
// Every page is read through a buffer resource whose base is that page's
// (page, kv head) block (64-bit address arithmetic, so pools may exceed
// 4 GB) and whose size is the block: an offset outside it reads zero.
// At head_dim <= 128 the K and V code loads are non-temporal (cache policy
// nt): a pass reads each page's codes once, and streaming them leaves the L2
// to what the kernels after attention read (measured: the whole pass
// 0.4-1.3% faster at 32 one-row chats and 0.7-0.8% at 16 verify jobs of 8
// rows, although the attention launch alone is slower). At head_dim 256 (one
// wave a SIMD) they measured 2-3% slower for the whole pass and stay
// ordinary loads, as do the 1 KiB scale blocks (non-temporal: no better).
//
// Every lane builds its fragments and rescales O on every page, with no
// branch on row state: MFMA reads all lanes' operands whatever the execution
// mask, and a still fully masked row (max -inf) just takes alpha = 0, p = 0.
// One work item of a wave: its (job, kv head, m-tile) over the chunk's pages,
// with the wave's LDS slices for the page's K and V scale blocks.
// Whether any of four V scales (f32 bits) is too large for the shifted P.V
// split (p * s * PV_SHIFT would overflow f16) — or not finite.
__device__ static inline bool pv_big(u32x4 v) {
    bool b = false;
#pragma unroll
    for (int e = 0; e < 4; e++) b = b || !(__uint_as_float(v[e]) <= PV_SCALE_MAX);
    return b;
}

template <int NG>
__device__ __forceinline__ void attn_item(const AttnItem& it, const uint4* __restrict__ Qp,
                                          const uint8_t* __restrict__ kpool, const uint8_t* __restrict__ vpool,
                                          const uint32_t* __restrict__ page_table, const KVGeom& g, int group,
                                          int ppw, float* __restrict__ part, float* ksl_w, float* vsl_w) {
    constexpr int D = 32 * NG;
    constexpr int DT = D / 16;
    constexpr int SCL = NG > 4 ? NG / 4 : 1;   // 1 KiB loads per scale block (16 B a lane)
    const int lane = threadIdx.x & 63, j4 = lane >> 4, l16 = lane & 15;
    const int T_act = it.past + it.n;
    const int R = it.n * group;
    const int npg = (T_act + 63) >> 6;
    const int p0 = it.p0;
    const int p1 = min(npg, p0 + ppw);
    const int mtq = it.mt;
    // scores in log2 units: exp(s/sqrt(D)) = exp2(s * log2(e)/sqrt(D)), one v_exp_f32 each
    const float score_scale = 1.4426950408889634f / sqrtf((float)D);

    uint4 qh[NG], ql[NG];
    {
        const size_t qb = (size_t)it.qb + lane;
#pragma unroll
        for (int gg = 0; gg < NG; gg++) {
            qh[gg] = Qp[qb + (size_t)gg * 128];
            ql[gg] = Qp[qb + (size_t)gg * 128 + 64];
        }
    }
    const int rho = mtq * 16 + l16;
    const int lim = rho < R ? it.past + rho / group : -1;   // last visible token of this row
    const uint32_t* pt = page_table + (size_t)it.slot * g.max_pages;
    const size_t hoff = (size_t)it.kvh * g.blk;
    const size_t pstride = (size_t)g.nKV * g.blk;
    // The chunk's page indices, one a lane (ppw <= 64): a page reads its own
    // with v_readlane, so no memory access sits on the page-to-page path.
    const uint32_t pgv = lane < p1 - p0 ? pt[p0 + lane] : 0u;
    auto page_rsrc = [&](const uint8_t* pool, int p) {
        const uint32_t pg = __builtin_amdgcn_readlane(pgv, p - p0);
        return __builtin_amdgcn_make_buffer_rsrc((void*)(pool + (size_t)pg * pstride + hoff), 0, g.blk, 0x00020000);
    };
    // Lane offsets inside a block (layout of k_fin_qkv's writes):
    const int vk = l16 * D + (D / 4) * j4;   // K codes: token row l16 of a 16-token tile, lane's k-block
    const int vv = j4 * D * 16 + l16 * 16;   // V codes: lane's token block, channel l16 of a d-tile
    // Scale blocks sit at 64*D in both blocks: K [64 tokens][NG], V [4][NG][16] at vpos.
    // The V scales go to LDS as [NG][4][16]: the four token blocks a wave reads
    // at once then sit in different banks. Each lane loads the 16 bytes it
    // stores at its own LDS offset, so the stores are contiguous as well.
    int vso[SCL];
#pragma unroll
    for (int q = 0; q < SCL; q++) {
        const int e = 256 * q + lane * 4, b = e >> 6, jb = (e >> 4) & 3;
        vso[q] = 4 * ((jb * NG + b) * 16 + (e & 15));
    }

    float mrow = -INFINITY, lsum = 0.0f;
    bool shifted = true;   // this row's p carries 2^PV_SHIFT_LOG2 (its O and lsum too) until dropped
    float4_t o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = float4_t{0.f, 0.f, 0.f, 0.f};

    u32x4 kc[4][NG / 2], vc[DT];
    u32x4 kst[SCL], vst[SCL];   // the next page's scale blocks, 16 B a lane per KiB, on their way to LDS
    // the next page's scale blocks, then its K codes
    auto load_k = [&](__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv) {
#pragma unroll
        for (int q = 0; q < SCL; q++) {
            kst[q] = __builtin_amdgcn_raw_buffer_load_b128(rk, lane * 16, 64 * D + 1024 * q, 0);
            vst[q] = __builtin_amdgcn_raw_buffer_load_b128(rv, vso[q], 64 * D, 0);
        }
#pragma unroll
        for (int tt = 0; tt < 4; tt++)
#pragma unroll
            for (int q = 0; q < NG / 2; q++)
                kc[tt][q] = __builtin_amdgcn_raw_buffer_load_b128(rk, vk, tt * 16 * D + 16 * q, NG > 4 ? 0 : 2);
    };
    auto load_v = [&](__amdgpu_buffer_rsrc_t rv) {
#pragma unroll
        for (int dt = 0; dt < DT; dt++) vc[dt] = __builtin_amdgcn_raw_buffer_load_b128(rv, vv, dt * 256, NG > 4 ? 0 : 2);
    };
    // One page. Its scale blocks arrived in kst/vst during the previous page;
    // they go to this wave's LDS slice first (a wave's LDS accesses run in
    // order, so the previous page's reads of the slice are done). The V
    // scales of tokens past the job's are another session's stale values
    // (even NaN): they go in as zero, so p * s is zero for every token whose
    // p is (a masked token's p is exp2(-inf) = +0, every scale of a visible
    // token is finite and positive).
    auto page = [&](int p) {
        // the last page reloads itself instead of branching (an L2 hit)
        const int pn = p + 1 < p1 ? p + 1 : p;
        bool big = false;
#pragma unroll
        for (int q = 0; q < SCL; q++) {
            *(u32x4*)&ksl_w[256 * q + lane * 4] = kst[q];
            u32x4 v = vst[q];
            if (p * 64 + 64 > T_act) {
                // LDS element 256q + 4 lane + e holds V position v = 16 jj + 4 (lane & 3) + e,
                // jj = ((256q + 4 lane) >> 4) & 3: the page's token vpos(v) = 16 (lane & 3) + 4 jj + e
                const int t0 = p * 64 + 16 * (lane & 3) + 4 * (((256 * q + lane * 4) >> 4) & 3);
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (t0 + e >= T_act) v[e] = 0u;
            }
            big = big || pv_big(v);
            *(u32x4*)&vsl_w[256 * q + lane * 4] = v;
        }
        const bool pbig = __builtin_amdgcn_ballot_w64(big) != 0;
        {
            float pr[4][4];
            float pm = -INFINITY;
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
                float ks[4 * NG];   // tokens 16tt + 4j4 + r, groups 0..NG-1
#pragma unroll
                for (int q = 0; q < NG; q++) {
                    const float4 f = *(const float4*)&ksl_w[(tt * 16 + 4 * j4) * NG + 4 * q];
                    ks[4 * q] = f.x; ks[4 * q + 1] = f.y; ks[4 * q + 2] = f.z; ks[4 * q + 3] = f.w;
                }
                float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int gg = 0; gg < NG; gg++) {
                    const u32x4 c = kc[tt][gg >> 1];
                    const half8_t kf = (gg & 1) ? dequant8_biased(c[2], c[3]) : dequant8_biased(c[0], c[1]);
                    float4_t pp = {0.f, 0.f, 0.f, 0.f};
                    pp = mfma16x16x32(kf, __builtin_bit_cast(half8_t, qh[gg]), pp);
                    pp = mfma16x16x32(kf, __builtin_bit_cast(half8_t, ql[gg]), pp);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(ks[r * NG + gg], pp[r], acc[r]);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) pr[tt][r] = acc[r] * score_scale;
            }
            // every token up to the job's first new position is visible to every
            // query row (and below T_act): only a page past it needs the per-cell
            // mask. The m-tile's lanes past the job's rows then carry unmasked
            // scores; they stay in their own lanes and MFMA columns, never written.
            if (p * 64 + 63 > it.past) {
#pragma unroll
                for (int tt = 0; tt < 4; tt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int tok = p * 64 + tt * 16 + 4 * j4 + r;
                        if (!(tok < T_act && tok <= lim)) pr[tt][r] = -INFINITY;
                    }
            }
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
#pragma unroll
                for (int r = 0; r < 4; r++) pm = fmaxf(pm, pr[tt][r]);
            const auto rvn = page_rsrc(vpool, pn);
            load_k(page_rsrc(kpool, pn), rvn);   // the K registers are free: start the next page
            __builtin_amdgcn_sched_barrier(0);
            pm = fmaxf(pm, __shfl_xor(pm, 16));
            pm = fmaxf(pm, __shfl_xor(pm, 32));
            const float mnew = fmaxf(mrow, pm);
            // the row drops the shift for good on a page whose V scales or its own
            // running max (in log2 units) leave no f16 room for p * s
            const bool drop = pbig || !(fabsf(mnew) < PV_MAX_SCORE);
            const float shrink = drop && shifted ? PV_UNSHIFT : 1.0f;
            shifted = shifted && !drop;
            const float alpha = (mrow == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrow - mnew)) * shrink;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++) o[dt][r] *= alpha;
            const float msub = (mnew == -INFINITY ? 0.0f : mnew) - (shifted ? PV_SHIFT_LOG2 : 0.0f);
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float e = __builtin_amdgcn_exp2f(pr[tt][r] - msub);   // masked: exp2(-inf) = 0
                    pr[tt][r] = e;
                    lsum += e;
                }
            __builtin_amdgcn_sched_barrier(0);
            // p * s (p times 2^PV_SHIFT_LOG2 while shifted) as hi + lo (split_hilo2), both into O
#pragma unroll
            for (int b = 0; b < NG; b++) {
                float sv[16];   // the lane's 16 tokens of 32-block b
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 f = *(const float4*)&vsl_w[b * 64 + 16 * j4 + 4 * q];
                    sv[4 * q] = f.x; sv[4 * q + 1] = f.y; sv[4 * q + 2] = f.z; sv[4 * q + 3] = f.w;
                }
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    u32x4 phw, plw;
#pragma unroll
                    for (int ii = 0; ii < 8; ii += 2) {
                        const int tt = 2 * ks + (ii >> 2), r = ii & 3;
                        const float p0 = pr[tt][r] * sv[4 * tt + r];
                        const float p1 = pr[tt][r + 1] * sv[4 * tt + r + 1];
                        uint32_t h, l;
                        split_hilo2(p0, p1, h, l);
                        phw[ii >> 1] = h;
                        plw[ii >> 1] = l;
                    }
                    const half8_t ph = __builtin_bit_cast(half8_t, phw), pl = __builtin_bit_cast(half8_t, plw);
#pragma unroll
                    for (int dd = 0; dd < 2; dd++) {
                        const int dt = 2 * b + dd;
                        const u32x4 c = vc[dt];
                        const half8_t vf = ks ? dequant8_biased(c[2], c[3]) : dequant8_biased(c[0], c[1]);
                        o[dt] = mfma16x16x32(vf, ph, o[dt]);
                        o[dt] = mfma16x16x32(vf, pl, o[dt]);
                    }
                }
            }
            mrow = mnew;
            load_v(rvn);
        }
    };
    if (p0 < p1) {
        const auto rv = page_rsrc(vpool, p0);
        load_k(page_rsrc(kpool, p0), rv);
        load_v(rv);
        for (int p = p0; p < p1; p++) page(p);
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    // partial row: max, sum, two pad floats, then O (16-byte aligned), the
    // shift taken off; rows past the job's R query rows are neither written
    // nor read
    if (rho < R) {
        const float un = shifted ? PV_UNSHIFT : 1.0f;
        float* dst = part + it.part + (size_t)l16 * (D + 4);
#pragma unroll
        for (int dt = 0; dt < DT; dt++) *(float4_t*)(dst + 4 + dt * 16 + 4 * j4) = o[dt] * un;
        if (j4 == 0) *(float2*)dst = make_float2(mrow, lsum * un);
    }
}


// One block of a job of several m-tiles: its four waves hold m-tiles
// 4b .. 4b+3 of one (job, kv head, chunk) (an m-tile past the job's is an
// empty slot, mt < 0) and read the same pages. Each wave loads a quarter of
// a page (K token tile w, V d-tiles w*DT/4 ..), dequantises it once into the
// workgroup's LDS, and every wave's MFMAs read the fragments from there, so a
// page is dequantised once instead of once per m-tile; a block with an empty
// slot has its idle wave 3 load and dequantise the whole page instead, while
// the other waves only compute. One barrier a page;
// the fragments are double-buffered (a wave past page p's barrier has
// finished page p - 1, so page p + 1 may reuse that buffer). Every value and
// every operation of a row is the one attn_item computes for it.
template <int NG>
__device__ __forceinline__ void attn_block4(const AttnItem& it, const AttnItem& it0, int wv,
                                            const uint4* __restrict__ Qp, const uint8_t* __restrict__ kpool,
                                            const uint8_t* __restrict__ vpool,
                                            const uint32_t* __restrict__ page_table, const KVGeom& g, int group,
                                            int ppw, float* __restrict__ part, u32x4* lds) {
    constexpr int D = 32 * NG;
    constexpr int DT = D / 16, DQ = DT / 4;
    constexpr int SCL = NG > 4 ? NG / 4 : 1;
    // LDS: K fragments [2][4 tt][NG gg][64], V fragments [2][DT][2 ks][64], then the
    // K and V scale blocks [2][256 * SCL] floats each, then the pages' range flags [2]
    u32x4* kf_s = lds;
    u32x4* vf_s = kf_s + 2 * 4 * NG * 64;
    float* ks_s = (float*)(vf_s + 2 * DT * 2 * 64);
    float* vs_s = ks_s + 2 * 256 * SCL;
    int* big_s = (int*)(vs_s + 2 * 256 * SCL);   // [2]: the page's V scales forbid the P.V shift
    const int lane = threadIdx.x & 63, j4 = lane >> 4, l16 = lane & 15;
    const int T_act = it0.past + it0.n;
    const int R = it0.n * group;
    const int npg = (T_act + 63) >> 6;
    const int p0 = it0.p0;
    const int p1 = min(npg, p0 + ppw);
    const bool mine = it.mt >= 0;
    const float score_scale = 1.4426950408889634f / sqrtf((float)D);

    uint4 qh[NG], ql[NG];
    if (mine) {
        const size_t qb = (size_t)it.qb + lane;
#pragma unroll
        for (int gg = 0; gg < NG; gg++) {
            qh[gg] = Qp[qb + (size_t)gg * 128];
            ql[gg] = Qp[qb + (size_t)gg * 128 + 64];
        }
    }
    const int rho = (mine ? it.mt : 0) * 16 + l16;
    const int lim = mine && rho < R ? it0.past + rho / group : -1;
    const uint32_t* pt = page_table + (size_t)it0.slot * g.max_pages;
    const size_t hoff = (size_t)it0.kvh * g.blk;
    const size_t pstride = (size_t)g.nKV * g.blk;
    const uint32_t pgv = lane < p1 - p0 ? pt[p0 + lane] : 0u;
    auto page_rsrc = [&](const uint8_t* pool, int p) {
        const uint32_t pg = __builtin_amdgcn_readlane(pgv, p - p0);
        return __builtin_amdgcn_make_buffer_rsrc((void*)(pool + (size_t)pg * pstride + hoff), 0, g.blk, 0x00020000);
    };
    const int vk = l16 * D + (D / 4) * j4;
    const int vv = j4 * D * 16 + l16 * 16;
    int vso[SCL];
#pragma unroll
    for (int q = 0; q < SCL; q++) {
        const int e = 256 * q + lane * 4, b = e >> 6, jb = (e >> 4) & 3;
        vso[q] = 4 * ((jb * NG + b) * 16 + (e & 15));
    }

    float mrow = -INFINITY, lsum = 0.0f;
    bool shifted = true;   // as in attn_item
    float4_t o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = float4_t{0.f, 0.f, 0.f, 0.f};

    // this wave's quarter of the next page: K token tile wv, V d-tiles wv*DQ .. +DQ-1,
    // and (waves 0 and 1) the K or V scale block
    u32x4 kc[NG / 2], vc[DQ], sc[SCL];
    auto load = [&](int p) {
        const auto rk = page_rsrc(kpool, p), rv = page_rsrc(vpool, p);
#pragma unroll
        for (int q = 0; q < NG / 2; q++) kc[q] = __builtin_amdgcn_raw_buffer_load_b128(rk, vk, wv * 16 * D + 16 * q, NG > 4 ? 0 : 2);
#pragma unroll
        for (int i = 0; i < DQ; i++) vc[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, vv, (wv * DQ + i) * 256, NG > 4 ? 0 : 2);
        if (wv == 0) {
#pragma unroll
            for (int q = 0; q < SCL; q++) sc[q] = __builtin_amdgcn_raw_buffer_load_b128(rk, lane * 16, 64 * D + 1024 * q, 0);
        } else if (wv == 1) {
#pragma unroll
            for (int q = 0; q < SCL; q++) sc[q] = __builtin_amdgcn_raw_buffer_load_b128(rv, vso[q], 64 * D, 0);
        }
    };
    // A block with an empty slot (a job of 3 m-tiles or fewer in its last
    // block, as a verify of 8 rows x 5 heads) gives its idle wave 3 the whole
    // page: it loads and dequantises everything, the same fragments the four
    // quarters would be, while the other waves only compute. Its page loop
    // has the same barriers as theirs.
    const int mtq = (it0.n * group + 15) >> 4;
    const bool spare = mtq - it0.mt < 4;
    if (spare && wv == 3) {
        u32x4 fk[4][NG / 2], fv[DT], fs[2][SCL];
        auto load_all = [&](int p) {
            const auto rk = page_rsrc(kpool, p), rv = page_rsrc(vpool, p);
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
#pragma unroll
                for (int q = 0; q < NG / 2; q++)
                    fk[tt][q] = __builtin_amdgcn_raw_buffer_load_b128(rk, vk, tt * 16 * D + 16 * q, NG > 4 ? 0 : 2);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) fv[dt] = __builtin_amdgcn_raw_buffer_load_b128(rv, vv, dt * 256, NG > 4 ? 0 : 2);
#pragma unroll
            for (int q = 0; q < SCL; q++) {
                fs[0][q] = __builtin_amdgcn_raw_buffer_load_b128(rk, lane * 16, 64 * D + 1024 * q, 0);
                fs[1][q] = __builtin_amdgcn_raw_buffer_load_b128(rv, vso[q], 64 * D, 0);
            }
        };
        if (p0 < p1) load_all(p0);
        for (int p = p0; p < p1; p++) {
            const int B = (p - p0) & 1;
            u32x4* kf = kf_s + B * 4 * NG * 64;
            u32x4* vf = vf_s + B * DT * 2 * 64;
            float* ksl = ks_s + B * 256 * SCL;
            float* vsl = vs_s + B * 256 * SCL;
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
#pragma unroll
                for (int q = 0; q < NG / 2; q++) {
                    kf[(tt * NG + 2 * q) * 64 + lane] = __builtin_bit_cast(u32x4, dequant8_biased(fk[tt][q][0], fk[tt][q][1]));
                    kf[(tt * NG + 2 * q + 1) * 64 + lane] =
                        __builtin_bit_cast(u32x4, dequant8_biased(fk[tt][q][2], fk[tt][q][3]));
                }
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                vf[(dt * 2) * 64 + lane] = __builtin_bit_cast(u32x4, dequant8_biased(fv[dt][0], fv[dt][1]));
                vf[(dt * 2 + 1) * 64 + lane] = __builtin_bit_cast(u32x4, dequant8_biased(fv[dt][2], fv[dt][3]));
            }
            bool big = false;
#pragma unroll
            for (int q = 0; q < SCL; q++) {
                *(u32x4*)&ksl[256 * q + lane * 4] = fs[0][q];
                u32x4 v = fs[1][q];
                if (p * 64 + 64 > T_act) {
                    const int t0 = p * 64 + 16 * (lane & 3) + 4 * (((256 * q + lane * 4) >> 4) & 3);
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (t0 + e >= T_act) v[e] = 0u;
                }
                big = big || pv_big(v);
                *(u32x4*)&vsl[256 * q + lane * 4] = v;
            }
            const bool pbig = __builtin_amdgcn_ballot_w64(big) != 0;
            if (lane == 0) big_s[B] = pbig ? 1 : 0;
            __syncthreads();
            if (p + 1 < p1) load_all(p + 1);
        }
        return;   // wave 3's slot is empty
    }
    if (p0 < p1 && !spare) load(p0);
    for (int p = p0; p < p1; p++) {
        const int B = (p - p0) & 1;
        u32x4* kf = kf_s + B * 4 * NG * 64;
        u32x4* vf = vf_s + B * DT * 2 * 64;
        float* ksl = ks_s + B * 256 * SCL;
        float* vsl = vs_s + B * 256 * SCL;
        if (!spare) {
#pragma unroll
            for (int q = 0; q < NG / 2; q++) {
                kf[(wv * NG + 2 * q) * 64 + lane] = __builtin_bit_cast(u32x4, dequant8_biased(kc[q][0], kc[q][1]));
                kf[(wv * NG + 2 * q + 1) * 64 + lane] = __builtin_bit_cast(u32x4, dequant8_biased(kc[q][2], kc[q][3]));
            }
#pragma unroll
            for (int i = 0; i < DQ; i++) {
                vf[((wv * DQ + i) * 2) * 64 + lane] = __builtin_bit_cast(u32x4, dequant8_biased(vc[i][0], vc[i][1]));
                vf[((wv * DQ + i) * 2 + 1) * 64 + lane] = __builtin_bit_cast(u32x4, dequant8_biased(vc[i][2], vc[i][3]));
            }
            if (wv == 0) {
#pragma unroll
                for (int q = 0; q < SCL; q++) *(u32x4*)&ksl[256 * q + lane * 4] = sc[q];
            } else if (wv == 1) {
                bool big = false;
#pragma unroll
                for (int q = 0; q < SCL; q++) {
                    u32x4 v = sc[q];
                    if (p * 64 + 64 > T_act) {   // stale scales past the job's tokens go in as zero
                        const int t0 = p * 64 + 16 * (lane & 3) + 4 * (((256 * q + lane * 4) >> 4) & 3);
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (t0 + e >= T_act) v[e] = 0u;
                    }
                    big = big || pv_big(v);
                    *(u32x4*)&vsl[256 * q + lane * 4] = v;
                }
                const bool pbig = __builtin_amdgcn_ballot_w64(big) != 0;
                if (lane == 0) big_s[B] = pbig ? 1 : 0;
            }
        }
        __syncthreads();
        if (p + 1 < p1 && !spare) load(p + 1);   // the registers are free: the next page is on its way
        if (!mine) continue;
        float pr[4][4];
        float pm = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            float ks[4 * NG];
#pragma unroll
            for (int q = 0; q < NG; q++) {
                const float4 f = *(const float4*)&ksl[(tt * 16 + 4 * j4) * NG + 4 * q];
                ks[4 * q] = f.x; ks[4 * q + 1] = f.y; ks[4 * q + 2] = f.z; ks[4 * q + 3] = f.w;
            }
            float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int gg = 0; gg < NG; gg++) {
                const half8_t kfr = __builtin_bit_cast(half8_t, kf[(tt * NG + gg) * 64 + lane]);
                float4_t pp = {0.f, 0.f, 0.f, 0.f};
                pp = mfma16x16x32(kfr, __builtin_bit_cast(half8_t, qh[gg]), pp);
                pp = mfma16x16x32(kfr, __builtin_bit_cast(half8_t, ql[gg]), pp);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(ks[r * NG + gg], pp[r], acc[r]);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) pr[tt][r] = acc[r] * score_scale;
        }
        // every token up to the job's first new position is visible to every
        // query row (and below T_act): only a page past it needs the per-cell
        // mask. The m-tile's lanes past the job's rows then carry unmasked
        // scores; they stay in their own lanes and MFMA columns, never written.
        if (p * 64 + 63 > it0.past) {
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int tok = p * 64 + tt * 16 + 4 * j4 + r;
                    if (!(tok < T_act && tok <= lim)) pr[tt][r] = -INFINITY;
                }
        }
#pragma unroll
        for (int tt = 0; tt < 4; tt++)
#pragma unroll
            for (int r = 0; r < 4; r++) pm = fmaxf(pm, pr[tt][r]);
        pm = fmaxf(pm, __shfl_xor(pm, 16));
        pm = fmaxf(pm, __shfl_xor(pm, 32));
        const float mnew = fmaxf(mrow, pm);
        const bool pbig = __builtin_amdgcn_readfirstlane(big_s[B]) != 0;
        const bool drop = pbig || !(fabsf(mnew) < PV_MAX_SCORE);   // as in attn_item
        const float shrink = drop && shifted ? PV_UNSHIFT : 1.0f;
        shifted = shifted && !drop;
        const float alpha = (mrow == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrow - mnew)) * shrink;
        lsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++) o[dt][r] *= alpha;
        const float msub = (mnew == -INFINITY ? 0.0f : mnew) - (shifted ? PV_SHIFT_LOG2 : 0.0f);
#pragma unroll
        for (int tt = 0; tt < 4; tt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float e = __builtin_amdgcn_exp2f(pr[tt][r] - msub);
                pr[tt][r] = e;
                lsum += e;
            }
#pragma unroll
        for (int b = 0; b < NG; b++) {
            float sv[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 f = *(const float4*)&vsl[b * 64 + 16 * j4 + 4 * q];
                sv[4 * q] = f.x; sv[4 * q + 1] = f.y; sv[4 * q + 2] = f.z; sv[4 * q + 3] = f.w;
            }
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                u32x4 phw, plw;
#pragma unroll
                for (int ii = 0; ii < 8; ii += 2) {
                    const int tt = 2 * ks + (ii >> 2), r = ii & 3;
                    uint32_t h, l;
                    split_hilo2(pr[tt][r] * sv[4 * tt + r], pr[tt][r + 1] * sv[4 * tt + r + 1], h, l);
                    phw[ii >> 1] = h;
                    plw[ii >> 1] = l;
                }
                const half8_t ph = __builtin_bit_cast(half8_t, phw), pl = __builtin_bit_cast(half8_t, plw);
#pragma unroll
                for (int dd = 0; dd < 2; dd++) {
                    const int dt = 2 * b + dd;
                    const half8_t vfr = __builtin_bit_cast(half8_t, vf[(dt * 2 + ks) * 64 + lane]);
                    o[dt] = mfma16x16x32(vfr, ph, o[dt]);
                    o[dt] = mfma16x16x32(vfr, pl, o[dt]);
                }
            }
        }
        mrow = mnew;
    }
    if (!mine) return;
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if (rho < R) {
        const float un = shifted ? PV_UNSHIFT : 1.0f;
        float* dst = part + it.part + (size_t)l16 * (D + 4);
#pragma unroll
        for (int dt = 0; dt < DT; dt++) *(float4_t*)(dst + 4 + dt * 16 + 4 * j4) = o[dt] * un;
        if (j4 == 0) *(float2*)dst = make_float2(mrow, lsum * un);
    }
}

// LDS of a k_attn workgroup: the four waves' scale slices for one-m-tile
// items (8 KiB per 4 groups), or a block's shared fragments and scales
// (attn_block4) when the launch holds jobs of several m-tiles (`multi`).
template <int NG>
constexpr size_t attn_lds_bytes() {
    constexpr size_t SCL = NG > 4 ? NG / 4 : 1, DT = 2 * NG;
    constexpr size_t single = 8 * 256 * SCL * 4;
    constexpr size_t block = (2 * 4 * NG * 64 + 2 * DT * 2 * 64) * 16 + 2 * 2 * 256 * SCL * 4 + 16;
    return single > block ? single : block;
}

// Work items go to waves in workgroups of four (item 4b + w to wave w of
// block b). Workgroup i takes block i; with `dyn` set, it then takes blocks
// gridDim.x, gridDim.x + 1, ... from the counter ctr[par] as it finishes
// each (launch_attn sets it for launches a little over one round of
// resident workgroups: dispatch hands a pending workgroup to a fixed XCD, so
// the few blocks past the first round would wait for that XCD's slowest
// workgroups). Each launch clears the counter of the next launch on its
// stream, ctr[par ^ 1]; the one it counts with was cleared by the
// launch before it. A block of one chunk's m-tiles (a job of several
// m-tiles, in a launch with `multi` set) runs attn_block4, its four waves
// sharing each page's dequantised fragments; other blocks' waves run their
// items on their own (attn_item).
template <int NG>
__global__ __launch_bounds__(256, NG > 4 ? 1 : 2) void k_attn(const AttnItem* __restrict__ items, int nitems,
                                                 const uint4* __restrict__ Qp,
                                                 const uint8_t* __restrict__ kpool, const uint8_t* __restrict__ vpool,
                                                 const uint32_t* __restrict__ page_table, KVGeom g, int group, int ppw,
                                                 float* __restrict__ part, uint32_t* __restrict__ ctr, int par,
                                                 int dyn, int multi) {
    // per wave, the current page's K and V scale blocks (64 tokens x NG groups,
    // f32), or a block's shared fragments: attn_lds_bytes<NG>() of dynamic LDS
    constexpr int SCL = NG > 4 ? NG / 4 : 1;
    extern __shared__ __attribute__((aligned(1024))) u32x4 lds[];
    __shared__ int s_blk;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(&ctr[par ^ 1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int nblk = (nitems + 3) / 4;
    for (int blk = blockIdx.x;;) {
        const int wid = blk * 4 + wv;
        const AttnItem it0 = items[blk * 4];
        if (multi && it0.n * group > 16) {
            // a job of several m-tiles: the block is one chunk's m-tiles (mt < 0 pads it)
            attn_block4<NG>(items[wid], it0, wv, Qp, kpool, vpool, page_table, g, group, ppw, part, lds);
        } else if (wid < nitems) {
            const AttnItem it = items[wid];
            if (it.mt >= 0)
                attn_item<NG>(it, Qp, kpool, vpool, page_table, g, group, ppw, part, (float*)lds + wv * 256 * SCL,
                              (float*)lds + (4 + wv) * 256 * SCL);
        }
        if (!dyn) break;   // no barriers then: a finished wave may leave
        __syncthreads();
        if (threadIdx.x == 0) s_blk = (int)gridDim.x + (int)atomicAdd(&ctr[par], 1u);
        __syncthreads();
        blk = s_blk;
        if (blk >= nblk) break;
    }
}

void launch_attn(hipStream_t st, const AttnItem* items, int nitems, const uint4* Qp,
                 const uint8_t* kpool, const uint8_t* vpool, const uint32_t* page_table, const KVGeom& g, int group,
                 int ppw, float* part, int multi, AttnSched& sc) {
    if (nitems <= 0) return;
    const int nblk = (nitems + 3) / 4;
    const int cap = sc.ncu * (g.ng == 8 ? 1 : 2);   // workgroups resident at once
    // blocks past the first round go out from the counter while they are few;
    // with more, dispatch's own rounds balance them
    const int dyn = nblk > cap && 2 * nblk <= 3 * cap;
    const int blocks = dyn ? cap : nblk;
    const int par = (int)(sc.seq++ & 1u);
    static bool attr = false;
    if (!attr) {
        attr = true;
        (void)hipFuncSetAttribute((const void*)k_attn<8>, hipFuncAttributeMaxDynamicSharedMemorySize, attn_lds_bytes<8>());
        (void)hipFuncSetAttribute((const void*)k_attn<4>, hipFuncAttributeMaxDynamicSharedMemorySize, attn_lds_bytes<4>());
        (void)hipFuncSetAttribute((const void*)k_attn<2>, hipFuncAttributeMaxDynamicSharedMemorySize, attn_lds_bytes<2>());
    }
    if (g.ng == 8)
        hipLaunchKernelGGL(k_attn<8>, dim3(blocks), dim3(256), multi ? attn_lds_bytes<8>() : 8 * 256 * 2 * 4, st, items, nitems, Qp, kpool, vpool, page_table, g,
                     group, ppw, part, sc.ctr, par, dyn, multi);
    else if (g.ng == 4)
        hipLaunchKernelGGL(k_attn<4>, dim3(blocks), dim3(256), multi ? attn_lds_bytes<4>() : 8 * 256 * 1 * 4, st, items, nitems, Qp, kpool, vpool, page_table, g,
                     group, ppw, part, sc.ctr, par, dyn, multi);
    else
        hipLaunchKernelGGL(k_attn<2>, dim3(blocks), dim3(256), multi ? attn_lds_bytes<2>() : 8 * 256 * 1 * 4, st, items, nitems, Qp, kpool, vpool, page_table, g,
                     group, ppw, part, sc.ctr, par, dyn, multi);
    CHECK_LAUNCH();
}

// Merge the chunk partials of one (job, kv head, m-tile): log-sum-exp over
// chunks, normalise, and write the merged-heads rows as the o_proj operand
// (merge_heads, web/model/kernels.js:1315-1329, is this indexing). Work item
// i's partial sits at part + i*16*(D + 4) (items are built in that order,
// chunk fastest). One wave per row takes the row's max and weighted sum
// across its lanes (a fixed butterfly order, so the bits depend only on the
// job's chunk count); the weights exp2(m_c - M) go to LDS. Then four groups
// of 256 threads each merge a quarter of the chunks (in order, eight chunks'
// loads in flight), one row's 8 columns a thread, and the quarters are added
// in order through LDS.
constexpr int COMBINE_CMAX = 512, COMBINE_SPLIT = 4;
template <int D>
__global__ __launch_bounds__(1024) void k_attn_combine(const JobDev* __restrict__ jobs, const float* __restrict__ part,
                                                       KVGeom g, int nH, int group, int KU, uint4* __restrict__ Xp,
                                                       float* __restrict__ ctx_out,
                                                       const int32_t* __restrict__ wg_job,
                                                       const float* __restrict__ gate) {
    // rows padded by one float: the four rows a wave reads at one chunk fall in
    // different banks; the quarters' halves in separate arrays, 16 B a thread
    __shared__ float wgt[16][COMBINE_CMAX + 1];
    __shared__ float Ls[16];
    __shared__ float4 red[COMBINE_SPLIT - 1][2][256];
    const int job = wg_job[3 * blockIdx.x], kvh = wg_job[3 * blockIdx.x + 1], mt = wg_job[3 * blockIdx.x + 2];
    const JobDev jb = jobs[job];
    constexpr int W = D + 4;
    const int R = jb.n * group;
    const int nc = jb.nchunk;
    const size_t pstride = (size_t)16 * W;
    const float* base = part + (size_t)(jb.item0 + (kvh * jb.mtq + mt) * nc) * pstride;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // 16 rows x D columns, 8 a thread, in chunks of at most 128 columns (one
    // chunk up to D = 128, two at D = 256); every thread reaches every barrier
    const int sub = threadIdx.x >> 8, t = threadIdx.x & 255;
    constexpr int CW = D < 128 ? D : 128, PRE = D > 128 ? 4 : 8;   // 8 at D = 256 spills at 128 VGPRs
    const int rl2 = t / (CW / 8);
    const bool live = rl2 < 16 && mt * 16 + rl2 < R;
    const int ca = (sub * nc) / COMBINE_SPLIT, c1 = ((sub + 1) * nc) / COMBINE_SPLIT;
    // the first PRE chunks' values of the first column chunk, loaded before
    // the weights are formed (they do not depend on them)
    float4 pa[PRE], pb[PRE];
    if (live) {
        const float* src = base + (size_t)rl2 * W + 4 + (t % (CW / 8)) * 8;
#pragma unroll
        for (int u = 0; u < PRE; u++)
            if (ca + u < c1) {
                pa[u] = *(const float4*)(src + (ca + u) * pstride);
                pb[u] = *(const float4*)(src + (ca + u) * pstride + 4);
            }
    }
    // only the m-tile's query rows rho < R were written (k_attn skips the rest)
    if (mt * 16 + wave < R) {
        const int rl = wave;   // 16 waves, one row each
        // (max, sum) of chunk `lane` loaded once; chunks past 64 in a loop
        const float2 ml0 = lane < nc ? *(const float2*)(base + lane * pstride + rl * W)
                                     : make_float2(-INFINITY, 0.0f);
        float mloc = ml0.x;
        for (int c = lane + 64; c < nc; c += 64) mloc = fmaxf(mloc, base[c * pstride + rl * W]);
        const float M = wave_max(mloc);
        float lloc = 0.0f;
        if (lane < nc) {
            const float w = ml0.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml0.x - M);
            wgt[rl][lane] = w;
            lloc += ml0.y * w;
        }
        for (int c = lane + 64; c < nc; c += 64) {
            const float2 ml = *(const float2*)(base + c * pstride + rl * W);
            const float w = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - M);
            wgt[rl][c] = w;
            lloc += ml.y * w;
        }
        const float L = wave_sum(lloc);
        if (lane == 0) Ls[rl] = L;
    }
    __syncthreads();
    const int rl = rl2;
    const int rho = mt * 16 + rl;
    for (int c0 = 0; c0 < D; c0 += CW) {
        const int d0 = c0 + (t % (CW / 8)) * 8;
        float O[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (live) {
            const float* src = base + (size_t)rl * W + 4 + d0;
            auto add = [&](const float4& a, const float4& b, float w) {
                O[0] += a.x * w; O[1] += a.y * w; O[2] += a.z * w; O[3] += a.w * w;
                O[4] += b.x * w; O[5] += b.y * w; O[6] += b.z * w; O[7] += b.w * w;
            };
            int c = ca;
            if (c0 == 0) {
#pragma unroll
                for (int u = 0; u < PRE; u++)
                    if (ca + u < c1) add(pa[u], pb[u], wgt[rl][ca + u]);
                c = ca + PRE < c1 ? ca + PRE : c1;
            }
            for (; c + 8 <= c1; c += 8) {
                float4 a[8], b[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    a[u] = *(const float4*)(src + (c + u) * pstride);
                    b[u] = *(const float4*)(src + (c + u) * pstride + 4);
                }
#pragma unroll
                for (int u = 0; u < 8; u++) add(a[u], b[u], wgt[rl][c + u]);
            }
            for (; c < c1; c++) add(*(const float4*)(src + c * pstride), *(const float4*)(src + c * pstride + 4), wgt[rl][c]);
            if (sub > 0) {
                red[sub - 1][0][t] = make_float4(O[0], O[1], O[2], O[3]);
                red[sub - 1][1][t] = make_float4(O[4], O[5], O[6], O[7]);
            }
        }
        __syncthreads();
        if (sub == 0 && live) {
#pragma unroll
            for (int q = 0; q < COMBINE_SPLIT - 1; q++) {
                const float4 a = red[q][0][t], b = red[q][1][t];
                O[0] += a.x; O[1] += a.y; O[2] += a.z; O[3] += a.w;
                O[4] += b.x; O[5] += b.y; O[6] += b.z; O[7] += b.w;
            }
            float v[8];
            const float L = Ls[rl];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = O[j] / L;
            const int i = rho / group, gi = rho % group;
            const int r = jb.row0 + i;
            const int k = (kvh * group + gi) * D + d0;
            if (gate) {
                // sigmoid_mul (kernels.js:1822-1839): s = 1/(1+exp(-gate)), s*a
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float sg = 1.0f / (1.0f + expf(-gate[(size_t)r * nH * D + k + j]));
                    v[j] = sg * v[j];
                }
            }
            if (ctx_out) {
#pragma unroll
                for (int j = 0; j < 8; j++) ctx_out[(size_t)r * nH * D + k + j] = v[j];
            }
            write_hilo(Xp, r, k / 8, KU, v);
        }
        if (c0 + CW < D) __syncthreads();   // `red` is reused by the next chunk
    }
}

void launch_attn_combine(hipStream_t st, const JobDev* jobs, const float* part, const KVGeom& g, int nH, int group,
                         int KU, uint4* Xp, float* ctx_out, const int32_t* wg_job, int nwg, const float* gate) {
    if (nwg <= 0) return;
    if (g.D == 256)
        hipLaunchKernelGGL(k_attn_combine<256>, dim3(nwg), dim3(1024), 0, st, jobs, part, g, nH, group, KU, Xp, ctx_out,
                           wg_job, gate);
    else if (g.D == 128)
        hipLaunchKernelGGL(k_attn_combine<128>, dim3(nwg), dim3(1024), 0, st, jobs, part, g, nH, group, KU, Xp, ctx_out,
                           wg_job, gate);
    else
        hipLaunchKernelGGL(k_attn_combine<64>, dim3(nwg), dim3(1024), 0, st, jobs, part, g, nH, group, KU, Xp, ctx_out,
                           wg_job, gate);
    CHECK_LAUNCH();
}

// =============================================================== embedding ===
// gather_embed_nopos_q8 (web/model/kernels.js:895-917) + round_f16 (the
// embedding rows are rounded like a block's output, stage.js:1365-1370);
// or, for a pass entering past position 0, the f16 rows handed in.
__global__ void k_embed(const int32_t* __restrict__ ids, const uint16_t* __restrict__ hidden, int T, int H,
                        const uint8_t* __restrict__ rec, int Nt, int KU, int P, int f32s, float* __restrict__ x,
                        int round, int nrows) {
    const int t = blockIdx.y;
    const int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T || h >= H) return;
    if (!ids) {
        x[(size_t)t * H + h] = half_value(hidden[(size_t)t * H + h]);
        return;
    }
    const int v = ids[t];
    if (v < 0 || v >= nrows) {   // a token outside a shorter table (the MTP's draft rows) reads zero
        x[(size_t)t * H + h] = 0.0f;
        return;
    }
    const int tile = v >> 4, u = h >> 6, lane = (v & 15) + 16 * ((h & 31) >> 3);
    const int byte = 8 * ((h & 63) >> 5) + (h & 7);
    const uint8_t* r = rec + lx_record(tile, u, KU, P, Nt);
    const int8_t q = (int8_t)(r[(tile & 1) * 1024 + lane * 16 + byte] ^ 0x80);
    const uint8_t* sp = r + 2048 + (v & 15) * 8 + (tile & 1) * 4;
    const float sc = f32s ? *(const float*)sp : half_value(*(const uint16_t*)(sp + ((h >> 5) & 1) * 2));
    const float e = (float)q * sc;
    x[(size_t)t * H + h] = round ? round_f16_value(e) : e;
}

void launch_embed(hipStream_t st, const int32_t* ids, const uint16_t* hidden, int T, const QTensor& wte,
                  float* x, int round) {
    dim3 grid((wte.K + 255) / 256, T);
    hipLaunchKernelGGL(k_embed, grid, dim3(256), 0, st, ids, hidden, T, wte.K, wte.codes, wte.Nt, wte.KU, wte.P,
                       wte.f32s, x, round, ids ? wte.N : 0);
    CHECK_LAUNCH();
}

// rows[r] = src[r] >= 0 ? x row src[r] : alt row (-1 - src[r]), H floats each:
// the MTP's hidden rows, the session's kept row first (stage.js:1408-1417).
__global__ void k_gather_rows(const float* __restrict__ x, const float* __restrict__ alt,
                              const int32_t* __restrict__ src, int T, int H, float* __restrict__ rows) {
    const int r = blockIdx.y;
    const int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= T || h >= H) return;
    const int s = src[r];
    rows[(size_t)r * H + h] = s >= 0 ? x[(size_t)s * H + h] : alt[(size_t)(-1 - s) * H + h];
}

void launch_gather_rows(hipStream_t st, const float* x, const float* alt, const int32_t* src, int T, int H,
                        float* rows) {
    if (T <= 0) return;
    hipLaunchKernelGGL(k_gather_rows, dim3((H + 255) / 256, T), dim3(256), 0, st, x, alt, src, T, H, rows);
    CHECK_LAUNCH();
}

// ==================================================================== top-k ===
// topk_stage / topkRows (web/model/kernels.js:1453-1507, :2129-2144): per row
// the best M (value, index) pairs, larger value first, ties to the lower
// index. Keys pack (order-preserving value bits, ~index) so a descending
// sort of 64-bit keys is that order; 4096 keys per workgroup are bitonic
// sorted in LDS and the best M kept, stage after stage until one workgroup's
// output is left.
__device__ static inline uint64_t topk_key(float v, uint32_t i) {
    uint32_t b = f2u(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)b << 32) | (uint64_t)(0xffffffffu - i);
}

constexpr int TOPK_CH = 4096;

// A head logit: the LM-head matmul's planes added in order.
__device__ static inline float plane_sum(const float* __restrict__ p, int planes, size_t stride, size_t i) {
    float v = p[i];
    for (int q = 1; q < planes; q++) v = v + p[q * stride + i];
    return v;
}

__global__ __launch_bounds__(256) void k_topk_stage(const float* __restrict__ logits, int planes,
                                                    const uint64_t* __restrict__ keys_in, int n, int M,
                                                    uint64_t* __restrict__ out) {
    const size_t stride = (size_t)gridDim.y * n;
    __shared__ uint64_t s[TOPK_CH];
    const int row = blockIdx.y;
    const int base = blockIdx.x * TOPK_CH;
    for (int k = threadIdx.x; k < TOPK_CH; k += 256) {
        const int i = base + k;
        uint64_t key = 0;
        if (i < n)
            key = logits ? topk_key(plane_sum(logits, planes, stride, (size_t)row * n + i), (uint32_t)i)
                         : keys_in[(size_t)row * n + i];
        s[k] = key;
    }
    __syncthreads();
    for (int size = 2; size <= TOPK_CH; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < TOPK_CH; i += 256) {
                const int l = i ^ stride;
                if (l > i) {
                    const bool desc = (i & size) == 0;
                    const uint64_t a = s[i], b = s[l];
                    if (desc ? (a < b) : (a > b)) {
                        s[i] = b;
                        s[l] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    const int groups = gridDim.x;
    for (int m = threadIdx.x; m < M; m += 256) out[(size_t)row * groups * M + (size_t)blockIdx.x * M + m] = s[m];
}

__global__ void k_topk_unpack(const uint64_t* __restrict__ keys, int rows, int M, float* __restrict__ vals,
                              uint32_t* __restrict__ ids) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * M) return;
    const uint64_t k = keys[i];
    uint32_t b = (uint32_t)(k >> 32);
    b = (b & 0x80000000u) ? (b & 0x7fffffffu) : ~b;
    vals[i] = u2f(b);
    ids[i] = 0xffffffffu - (uint32_t)(k & 0xffffffffu);
}

// M = 1 (greedy, argmax_rows semantics: web/model/kernels.js:1411-1443): the
// largest key of 4096 entries per workgroup, then of the workgroups' keys.
__global__ __launch_bounds__(256) void k_argmax_stage(const float* __restrict__ logits, int planes,
                                                      const uint64_t* __restrict__ keys_in, int n,
                                                      uint64_t* __restrict__ out) {
    const size_t stride = (size_t)gridDim.y * n;
    __shared__ uint64_t red[256];
    const int row = blockIdx.y;
    const int base = blockIdx.x * TOPK_CH;
    uint64_t best = 0;
    for (int k = threadIdx.x; k < TOPK_CH; k += 256) {
        const int i = base + k;
        if (i >= n) break;
        const uint64_t key = logits ? topk_key(plane_sum(logits, planes, stride, (size_t)row * n + i), (uint32_t)i)
                                    : keys_in[(size_t)row * n + i];
        best = key > best ? key : best;
    }
    red[threadIdx.x] = best;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] = red[threadIdx.x + s] > red[threadIdx.x] ? red[threadIdx.x + s] : red[threadIdx.x];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[(size_t)row * gridDim.x + blockIdx.x] = red[0];
}

void launch_topk(hipStream_t st, const float* logits, int planes, int rows, int V, int M, uint64_t* a,
                 uint64_t* b, float* vals, uint32_t* ids) {
    if (M == 1) {
        int n = V;
        const float* lg = logits;
        const uint64_t* in = nullptr;
        uint64_t* out = a;
        uint64_t* other = b;
        for (;;) {
            const int groups = (n + TOPK_CH - 1) / TOPK_CH;
            hipLaunchKernelGGL(k_argmax_stage, dim3(groups, rows), dim3(256), 0, st, lg, planes, in, n, out);
            CHECK_LAUNCH();
            if (groups == 1) break;
            lg = nullptr;
            in = out;
            n = groups;
            uint64_t* t = out;
            out = other;
            other = t;
        }
        hipLaunchKernelGGL(k_topk_unpack, dim3((rows + 255) / 256), dim3(256), 0, st, out, rows, 1, vals, ids);
        CHECK_LAUNCH();
        return;
    }
    int n = V;
    const float* lg = logits;
    const uint64_t* in = nullptr;
    uint64_t* out = a;
    uint64_t* other = b;
    for (;;) {
        const int groups = (n + TOPK_CH - 1) / TOPK_CH;
        hipLaunchKernelGGL(k_topk_stage, dim3(groups, rows), dim3(256), 0, st, lg, planes, in, n, M, out);
        CHECK_LAUNCH();
        if (groups == 1) break;
        lg = nullptr;
        in = out;
        n = groups * M;
        uint64_t* t = out;
        out = other;
        other = t;
    }
    hipLaunchKernelGGL(k_topk_unpack, dim3((rows * M + 255) / 256), dim3(256), 0, st, out, rows, M, vals, ids);
    CHECK_LAUNCH();
}

// The staged keys launch_topk needs for (rows, V, M): the first half (`a`,
// stages 1, 3, ...) and the second (`b`, stages 2, 4, ...), in keys.
void topk_stage_keys(int rows, int V, int M, size_t* a_keys, size_t* b_keys) {
    size_t sa = 0, sb = 0;
    int n = V;
    for (bool to_a = true;; to_a = !to_a) {
        const int groups = (n + TOPK_CH - 1) / TOPK_CH;
        const size_t k = (size_t)rows * groups * M;
        if (to_a) sa = std::max(sa, k);
        else sb = std::max(sb, k);
        if (groups == 1) break;
        n = M == 1 ? groups : groups * M;
    }
    *a_keys = sa;
    *b_keys = sb;
}

// Scratch of the allocation-free top-k entry point (cc_topk_noalloc): the
// staged keys, both halves. Each GPU the library runs on holds its own copy
// until the process ends. Every key a stage reads was written by the stage
// before it in the same call, so nothing in it needs clearing between calls.
// In host code `scratch` names a host-side stand-in, never device memory:
// kernels get the per-device address topk_scratch_setup() looks up.
static __device__ __align__(256) uint64_t scratch[TOPK_SCRATCH_KEYS];

hipError_t topk_scratch_setup(int device, uint64_t** out) {
    static std::mutex mu;
    static uint64_t* ptrs[TOPK_SCRATCH_DEVICES] = {};
    if (device < 0 || device >= TOPK_SCRATCH_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[device]) {
        uint64_t* p = nullptr;
        const hipError_t e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        ptrs[device] = p;
    }
    *out = ptrs[device];
    return hipSuccess;
}

// ============================================================ small kernels ===
__global__ void k_round_f16(float* a, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        a[i] = round_f16_value(a[i]);
}

void launch_round_f16(hipStream_t st, float* a, int64_t n) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_round_f16, dim3((unsigned)blocks), dim3(256), 0, st, a, n);
    CHECK_LAUNCH();
}

__global__ void k_fill(float* p, int64_t n, float v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

void launch_fill(hipStream_t st, float* p, int64_t n, float v) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_fill, dim3((unsigned)blocks), dim3(256), 0, st, p, n, v);
    CHECK_LAUNCH();
}

// Page allocation (web/model/model.js:191-202 ensurePages, replayed for every
// job of the pass in job order): plan[4j..4j+3] = slot, owned, new, prefix.
// The host tracks counts (the stack top and each frame's length); the device
// holds the indices. Job j's k-th new page is the stack entry
// top-1-(prefix+k): what sequential pops would return.
__global__ void k_alloc_pages(const int32_t* __restrict__ plan, int njobs, const uint32_t* __restrict__ free_stack,
                              int top, uint32_t* __restrict__ page_table, int max_pages) {
    const int j = blockIdx.x;
    if (j >= njobs) return;
    const int slot = plan[4 * j], owned = plan[4 * j + 1], nw = plan[4 * j + 2], pre = plan[4 * j + 3];
    for (int k = threadIdx.x; k < nw; k += blockDim.x)
        page_table[(size_t)slot * max_pages + owned + k] = free_stack[top - 1 - (pre + k)];
}

void launch_alloc_pages(hipStream_t st, const int32_t* plan, int njobs, const uint32_t* free_stack, int top,
                        uint32_t* page_table, int max_pages) {
    if (njobs <= 0) return;
    hipLaunchKernelGGL(k_alloc_pages, dim3(njobs), dim3(64), 0, st, plan, njobs, free_stack, top, page_table,
                       max_pages);
    CHECK_LAUNCH();
}

// The next pass's ids from this pass's top-M output: column 0 (the greedy
// token) of each sampled row.
__global__ void k_ids_col0(const uint32_t* __restrict__ ids, int rows, int stride, int32_t* __restrict__ out) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) out[r] = (int32_t)ids[(size_t)r * stride];
}

void launch_ids_col0(hipStream_t st, const uint32_t* ids, int rows, int stride, int32_t* out) {
    if (rows <= 0) return;
    hipLaunchKernelGGL(k_ids_col0, dim3((rows + 255) / 256), dim3(256), 0, st, ids, rows, stride, out);
    CHECK_LAUNCH();
}

// ================================================================ packing ===
// One workgroup: per-job counts in parallel, their prefix sums in job order
// (pack_exscan), then every job's tables written by one wave, four jobs at a
// time. A job of n rows at past p needs ceil(n*group/16)
// Q m-tiles, ceil(ceil((p+n)/64)/ppw) chunks of pages per (kv head, m-tile),
// one combine triple per (kv head, m-tile), and nKV*mtq*ng*128 Q-operand
// units; each work item's softmax partial takes 16*(D+4) floats, at the
// item's index in (job, kv head, m-tile, chunk) order. The item list itself
// holds the jobs of several m-tiles first, each (kv head, chunk) as blocks of
// four m-tiles (padded with mt = -1), so one workgroup's four waves read the
// same pages together and the pages come from HBM once; then the jobs of
// one m-tile: first every chunk of ppw pages, then the last, shorter chunks,
// so the blocks a launch hands out last are the short ones (k_attn).
constexpr int PACK_THREADS = 256;

static_assert(PACK_MAX_JOBS <= 4 * PACK_THREADS, "pack_exscan takes four jobs a thread");
// Exclusive prefix sums of v[0 .. n) in place, n <= 4 * PACK_THREADS, over the
// whole workgroup (four consecutive values a thread, a wave scan, the waves'
// totals in order); `total` = the sum of all n. part: PACK_THREADS / 64 ints.
__device__ static void pack_exscan(int32_t* v, int n, int32_t* part, int& total) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    int a[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a[i] = 4 * t + i < n ? v[4 * t + i] : 0;
        s += a[i];
    }
    int x = s;   // inclusive scan of the threads' sums across the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == 63) part[w] = x;
    __syncthreads();
    int off = 0;
    total = 0;
#pragma unroll
    for (int k = 0; k < PACK_THREADS / 64; k++) {
        off += k < w ? part[k] : 0;
        total += part[k];
    }
    int run = off + x - s;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (4 * t + i < n) v[4 * t + i] = run;
        run += a[i];
    }
    __syncthreads();   // part is reused by the next scan
}

__global__ __launch_bounds__(PACK_THREADS) void k_pack(const PackJob* __restrict__ in, int njobs, int step,
                                                       PackGeom g, JobDev* __restrict__ jobs,
                                                       AttnItem* __restrict__ items, int32_t* __restrict__ row_job,
                                                       int32_t* __restrict__ head_rows, int32_t* __restrict__ cwg) {
    __shared__ int32_t s_row0[PACK_MAX_JOBS], s_item0[PACK_MAX_JOBS], s_cwg0[PACK_MAX_JOBS],
        s_qp0[PACK_MAX_JOBS], s_head0[PACK_MAX_JOBS], s_mtq[PACK_MAX_JOBS], s_nch[PACK_MAX_JOBS],
        s_pos0[PACK_MAX_JOBS], s_posf[PACK_MAX_JOBS], s_posb[PACK_MAX_JOBS], s_part[PACK_THREADS / 64];
    // each job's counts, then their exclusive prefix sums in job order
    for (int j = threadIdx.x; j < njobs; j += blockDim.x) {
        const int n = in[j].n, tact = in[j].past + step + n;
        const int mtq = (n * g.group + 15) / 16, pages = (tact + g.page - 1) / g.page;
        const int nch = (pages + g.ppw - 1) / g.ppw;
        s_mtq[j] = mtq;
        s_nch[j] = nch;
        s_row0[j] = n;
        s_item0[j] = g.nKV * mtq * nch;
        s_cwg0[j] = g.nKV * mtq;
        s_qp0[j] = g.nKV * mtq * g.ng * 128;
        s_head0[j] = g.head ? in[j].sampled : 0;
        // the item list: jobs of several m-tiles first, then the one-m-tile jobs'
        // full chunks, then their short last chunks
        s_pos0[j] = mtq > 1 ? g.nKV * nch * 4 * ((mtq + 3) / 4) : 0;
        s_posf[j] = mtq > 1 ? 0 : g.nKV * (pages / g.ppw);
        s_posb[j] = mtq > 1 ? 0 : g.nKV * (pages % g.ppw != 0);
    }
    __syncthreads();
    int tot_multi, tot_full, unused;
    pack_exscan(s_row0, njobs, s_part, unused);
    pack_exscan(s_item0, njobs, s_part, unused);
    pack_exscan(s_cwg0, njobs, s_part, unused);
    pack_exscan(s_qp0, njobs, s_part, unused);
    pack_exscan(s_head0, njobs, s_part, unused);
    pack_exscan(s_pos0, njobs, s_part, tot_multi);
    pack_exscan(s_posf, njobs, s_part, tot_full);
    pack_exscan(s_posb, njobs, s_part, unused);
    for (int j = threadIdx.x; j < njobs; j += blockDim.x)
        if (s_mtq[j] == 1) {
            s_pos0[j] = tot_multi + s_posf[j];
            s_posb[j] += tot_multi + tot_full;
        }
    __syncthreads();
    const int part = 16 * (g.D + 4);
    // one wave a job: the four waves write four jobs' tables at a time
    const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
    for (int j = wv; j < njobs; j += PACK_THREADS / 64) {
        const PackJob pj = in[j];
        const int past = pj.past + step, mtq = s_mtq[j], nch = s_nch[j];
        if (ln == 0) {
            JobDev jd;
            jd.slot = pj.slot;
            jd.past = past;
            jd.n = pj.n;
            jd.row0 = s_row0[j];
            jd.qp_off = s_qp0[j];
            jd.mtq = mtq;
            jd.item0 = s_item0[j];
            jd.nchunk = nch;
            jd.snap = pj.snap;
            jd.keep = pj.keep;
            jobs[j] = jd;
        }
        if (mtq == 1) {
            const int nfull = ((past + pj.n + g.page - 1) / g.page) / g.ppw;
            for (int x = ln; x < g.nKV * nch; x += 64) {
                const int c = x % nch, h = x / nch;
                const int idx = s_item0[j] + x;   // (kv head, m-tile 0, chunk)
                items[c < nfull ? s_pos0[j] + h * nfull + c : s_posb[j] + h] =
                    AttnItem{pj.slot, past, pj.n, 0, s_qp0[j] + (h * g.ng) * 128, idx * part, h, c * g.ppw};
            }
        } else {
            // (kv head, chunk, block of 4 m-tiles, m-tile): a block is one workgroup
            const int nb = (mtq + 3) / 4, nit = g.nKV * nch * nb * 4;
            for (int x = ln; x < nit; x += 64) {
                const int q = x % 4, b = (x / 4) % nb, c = (x / (4 * nb)) % nch, h = x / (4 * nb * nch);
                const int mt = 4 * b + q;
                if (mt >= mtq) {
                    items[s_pos0[j] + x] = AttnItem{0, 0, 0, -1, 0, 0, 0, 0};
                    continue;
                }
                const int hm = h * mtq + mt;
                const int idx = s_item0[j] + hm * nch + c;
                items[s_pos0[j] + x] =
                    AttnItem{pj.slot, past, pj.n, mt, s_qp0[j] + (hm * g.ng) * 128, idx * part, h, c * g.ppw};
            }
        }
        for (int x = ln; x < g.nKV * mtq; x += 64) {
            const int at = 3 * (s_cwg0[j] + x);
            cwg[at] = j;
            cwg[at + 1] = x / mtq;
            cwg[at + 2] = x % mtq;
        }
        for (int i = ln; i < pj.n; i += 64) row_job[s_row0[j] + i] = j;
        if (g.head)
            for (int i = ln; i < pj.sampled; i += 64)
                head_rows[s_head0[j] + i] = s_row0[j] + pj.n - pj.sampled + i;
    }
}

void launch_pack(hipStream_t st, const PackJob* in, int njobs, int step, const PackGeom& g, JobDev* jobs,
                 AttnItem* items, int32_t* row_job, int32_t* head_rows, int32_t* cwg) {
    if (njobs <= 0 || njobs > PACK_MAX_JOBS) return;
    hipLaunchKernelGGL(k_pack, dim3(1), dim3(PACK_THREADS), 0, st, in, njobs, step, g, jobs, items, row_job,
                       head_rows, cwg);
    CHECK_LAUNCH();
}

// freePages (web/model/model.js:204-211): push the frame's pages back, last
// owned first, so the next pop returns its first page.
__global__ void k_release_pages(int slot, int owned, uint32_t* __restrict__ free_stack, int top,
                                const uint32_t* __restrict__ page_table, int max_pages) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < owned; i += gridDim.x * blockDim.x)
        free_stack[top + i] = page_table[(size_t)slot * max_pages + owned - 1 - i];
}

void launch_release_pages(hipStream_t st, int slot, int owned, uint32_t* free_stack, int top,
                          const uint32_t* page_table, int max_pages) {
    if (owned <= 0) return;
    hipLaunchKernelGGL(k_release_pages, dim3((owned + 255) / 256), dim3(256), 0, st, slot, owned, free_stack,
                       top, page_table, max_pages);
    CHECK_LAUNCH();
}

// ================================================================ synthetic ===
// A q8 tensor [N, K] generated straight into the tiled layout at row tile
// `row_tile0` of w (fused tensors stack their row tiles). Codes
// clamp(round(N(0,40)), ±127) from the Irwin-Hall generator at index n*K + k;
// f16 scales ~U(1e-4, 4e-4) at index n*ng + g in stream ^ 0x5ca1e.
__global__ void k_gen_q8(uint8_t* __restrict__ rec, int Nt, int KU, int P, int row_tile0, int N, int K,
                         uint64_t seed, uint64_t stream) {
    const int tiles = (N + 15) / 16;
    const int64_t total = (int64_t)tiles * KU * 64;
    const int ng = (K + 31) / 32;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i & 63);
        const int64_t tu = i >> 6;
        const int u = (int)(tu % KU), t = (int)(tu / KU);
        const int n = 16 * t + (lane & 15);
        const int tg = row_tile0 + t;
        uint8_t* r = rec + lx_record(tg, u, KU, P, Nt);
        uint8_t b[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int k = 64 * u + 32 * (j >> 3) + 8 * (lane >> 4) + (j & 7);
            int q = 0;
            if (n < N && k < K) q = gen_code(cc_rng(seed, stream, (uint64_t)n * K + k));
            b[j] = (uint8_t)((q & 0xff) ^ 0x80);
        }
        uint8_t* dst = r + (tg & 1) * 1024 + lane * 16;
#pragma unroll
        for (int j = 0; j < 16; j++) dst[j] = b[j];
        if (lane < 16) {
            for (int h = 0; h < 2; h++) {
                const int gg = 2 * u + h;
                uint16_t sbits = 0;
                if (n < N && gg < ng) sbits = gen_scale_f16(seed, stream ^ 0x5ca1eull, (uint64_t)n * ng + gg, 1e-4, 4e-4);
                *(uint16_t*)(r + 2048 + lane * 8 + (tg & 1) * 4 + h * 2) = sbits;
            }
        }
    }
}

void launch_gen_q8(hipStream_t st, const QTensor& w, int row_tile0, int N, int K, uint64_t seed,
                   uint64_t stream) {
    const int64_t total = (int64_t)((N + 15) / 16) * w.KU * 64;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_gen_q8, dim3((unsigned)blocks), dim3(256), 0, st, w.codes, w.Nt, w.KU, w.P, row_tile0,
                       N, K, seed, stream);
    CHECK_LAUNCH();
}

// Host int8 [N, K] codes + scales -> records: f16 scales [N, ceil(K/32)]
// (f32s = 0), or f32 scales [N, KU], one per 64-wide unit (f32s = 1).
__global__ void k_tile_q8(const int8_t* __restrict__ src, const void* __restrict__ scv, int N, int K,
                          uint8_t* __restrict__ rec, int Nt, int KU, int P, int row_tile0, int f32s) {
    const int tiles = (N + 15) / 16;
    const int64_t total = (int64_t)tiles * KU * 64;
    const int ng = (K + 31) / 32;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i & 63);
        const int64_t tu = i >> 6;
        const int u = (int)(tu % KU), t = (int)(tu / KU);
        const int n = 16 * t + (lane & 15);
        const int tg = row_tile0 + t;
        uint8_t* r = rec + lx_record(tg, u, KU, P, Nt);
        uint8_t* dst = r + (tg & 1) * 1024 + lane * 16;
        for (int j = 0; j < 16; j++) {
            const int k = 64 * u + 32 * (j >> 3) + 8 * (lane >> 4) + (j & 7);
            const int q = (n < N && k < K) ? src[(size_t)n * K + k] : 0;
            dst[j] = (uint8_t)((q & 0xff) ^ 0x80);
        }
        if (lane < 16 && f32s) {
            const float* sc = (const float*)scv;
            *(float*)(r + 2048 + lane * 8 + (tg & 1) * 4) = n < N ? sc[(size_t)n * KU + u] : 0.0f;
        } else if (lane < 16) {
            const uint16_t* sc = (const uint16_t*)scv;
            for (int h = 0; h < 2; h++) {
                const int gg = 2 * u + h;
                *(uint16_t*)(r + 2048 + lane * 8 + (tg & 1) * 4 + h * 2) =
                    (n < N && gg < ng) ? sc[(size_t)n * ng + gg] : (uint16_t)0;
            }
        }
    }
}

void launch_tile_q8(hipStream_t st, const int8_t* codes, const void* scales, int N, int K, const QTensor& w,
                    int row_tile0) {
    const int64_t total = (int64_t)((N + 15) / 16) * w.KU * 64;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_tile_q8, dim3((unsigned)blocks), dim3(256), 0, st, codes, scales, N, K, w.codes, w.Nt,
                       w.KU, w.P, row_tile0, w.f32s);
    CHECK_LAUNCH();
}

// Random KV rows 0..tokens-1 of a slot in one layer's pool (which: 0 = K,
// 1 = V): the generator of the test oracle (codes uniform in ±127 at index
// base*D + d, base = ((key << 24) + t)*nKV + head; one f16 scale
// ~U(0.005, 0.02) at base, replicated into every 32-block).
__global__ void k_fill_kv(uint8_t* __restrict__ pool, const uint32_t* __restrict__ page_table, int slot,
                          int tokens, KVGeom g, uint64_t seed, uint64_t stream, uint64_t key, int which) {
    const int D = g.D;
    const int64_t total = (int64_t)tokens * g.nKV * D;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int d = (int)(i % D);
        const int64_t tn = i / D;
        const int n = (int)(tn % g.nKV), t = (int)(tn / g.nKV);
        const uint64_t base = ((key << 24) + (uint64_t)t) * (uint64_t)g.nKV + (uint64_t)n;
        const uint64_t r = cc_rng(seed, stream, base * (uint64_t)D + (uint64_t)d);
        const int8_t code = (int8_t)((int)((r >> 8) % 255u) - 127);
        const uint32_t page = page_table[(size_t)slot * g.max_pages + t / g.page];
        const int s = t % g.page;
        uint8_t* blk = pool + ((size_t)page * g.nKV + n) * g.blk;
        const uint8_t biased = (uint8_t)((uint8_t)code ^ 0x80u);
        if (which == 0) blk[(size_t)s * D + kpos(d, D)] = biased;
        else blk[vcode_at(d, s, D)] = biased;
        if ((d & 31) == 0) {
            const float sc = half_value(gen_scale_f16(seed, stream ^ 0x5ca1eull, base, 0.005, 0.02));
            const int b = d >> 5;
            if (which == 0) *(float*)(blk + 64 * D + ((size_t)s * g.ng + b) * 4) = sc;
            else *(float*)(blk + 64 * D + (size_t)vscale_at(b, s, g.ng) * 4) = sc;
        }
    }
}

void launch_fill_kv(hipStream_t st, uint8_t* pool, const uint32_t* page_table, int slot, int tokens,
                    const KVGeom& g, uint64_t seed, uint64_t stream, uint64_t key, int which) {
    const int64_t total = (int64_t)tokens * g.nKV * g.D;
    if (total <= 0) return;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_fill_kv, dim3((unsigned)blocks), dim3(256), 0, st, pool, page_table, slot, tokens, g,
                       seed, stream, key, which);
    CHECK_LAUNCH();
}

// Device block layout <-> the reference's rows (kernels.js:999-1022): row
// word w < D/4 packs codes 4w..4w+3 (low byte first, signed: the pool's
// biased bytes ^ 0x80); then D/32 f32 scales.
__global__ void k_kv_ref(uint8_t* __restrict__ pool, const uint32_t* __restrict__ page_table, int slot, int head,
                         int t0, int t1, KVGeom g, int which, uint32_t* __restrict__ rows, int to_ref) {
    const int D = g.D, RW = D / 4 + g.ng;
    const int64_t total = (int64_t)(t1 - t0) * RW;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int w = (int)(i % RW), t = t0 + (int)(i / RW);
        const uint32_t page = page_table[(size_t)slot * g.max_pages + t / g.page];
        const int s = t % g.page;
        uint8_t* blk = pool + ((size_t)page * g.nKV + head) * g.blk;
        if (w < D / 4) {
            uint8_t* p[4];
            for (int j = 0; j < 4; j++) {
                const int d = 4 * w + j;
                p[j] = which == 0 ? blk + (size_t)s * D + kpos(d, D) : blk + vcode_at(d, s, D);
            }
            if (to_ref) {
                uint32_t word = 0;
                for (int j = 0; j < 4; j++) word |= (uint32_t)(*p[j] ^ 0x80u) << (8 * j);
                rows[i] = word;
            } else {
                const uint32_t word = rows[i];
                for (int j = 0; j < 4; j++) *p[j] = (uint8_t)((word >> (8 * j)) ^ 0x80u);
            }
        } else {
            const int b = w - D / 4;
            uint32_t* sp = which == 0 ? (uint32_t*)(blk + 64 * D + ((size_t)s * g.ng + b) * 4)
                                      : (uint32_t*)(blk + 64 * D + (size_t)vscale_at(b, s, g.ng) * 4);
            if (to_ref) rows[i] = *sp;
            else *sp = rows[i];
        }
    }
}

void launch_kv_to_ref(hipStream_t st, const uint8_t* pool, const uint32_t* page_table, int slot, int head, int t0,
                      int t1, const KVGeom& g, int which, uint32_t* out) {
    const int64_t total = (int64_t)(t1 - t0) * (g.D / 4 + g.ng);
    if (total <= 0) return;
    hipLaunchKernelGGL(k_kv_ref, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, (uint8_t*)pool,
                       page_table, slot, head, t0, t1, g, which, out, 1);
    CHECK_LAUNCH();
}

void launch_kv_from_ref(hipStream_t st, uint8_t* pool, const uint32_t* page_table, int slot, int head, int t0,
                        int t1, const KVGeom& g, int which, const uint32_t* in) {
    const int64_t total = (int64_t)(t1 - t0) * (g.D / 4 + g.ng);
    if (total <= 0) return;
    hipLaunchKernelGGL(k_kv_ref, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, pool, page_table, slot,
                       head, t0, t1, g, which, (uint32_t*)in, 0);
    CHECK_LAUNCH();
}

// Sum the K splits of a projection: out[m][n] = sum_s part[s][m][n], in order.
__global__ void k_sum_splits(const float* __restrict__ part, int splits, int M, int N, float* __restrict__ out) {
    const int64_t total = (int64_t)M * N;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        float p = part[i];
        for (int s = 1; s < splits; s++) p = p + part[(size_t)s * total + i];
        out[i] = p;
    }
}

void launch_sum_splits(hipStream_t st, const float* part, int splits, int M, int N, float* out) {
    const int64_t total = (int64_t)M * N;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_sum_splits, dim3((unsigned)blocks), dim3(256), 0, st, part, splits, M, N, out);
    CHECK_LAUNCH();
}

// Rows of f16 values kept as f32 -> their half bits (exact).
__global__ void k_to_half_bits(const float* __restrict__ x, int64_t n, uint16_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = half_bits(x[i]);
}

void launch_to_half_bits(hipStream_t st, const float* x, int64_t n, uint16_t* out) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_to_half_bits, dim3((unsigned)blocks), dim3(256), 0, st, x, n, out);
    CHECK_LAUNCH();
}
