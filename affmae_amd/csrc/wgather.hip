// Weighted neighbour gathers for gfx950: the AFF downsampling merge.
//
//   weighted_features  OUT[b,i,ic,c] = sum_m W[b,i,m,ic] * F[b, idx[b,i,m], c]
//                      (reference src/layers/kernels/weighted_features.py:30-111)
//   weighted_gather    OUT[b,i,c]    = sum_m W[b,i,m] * F[b, idx[b,i,m], c]
//                      (reference src/layers/kernels/weighted_gather.py:21-102; the IC = 1 case)
//   softmax merge      w = softmax_m(-|p_i - p_idx| / tau); OUT = sum_m w F[idx], POS = sum_m w p[idx]
//                      (composition of knn + softmax + weighted_gather, fused)
//
// All accumulate in fp32 and store in the feature dtype.  Each output row is
// owned by a group of lanes (8 channels per lane, 16-byte loads); the group
// walks its neighbours 8 at a time with every gather issued before use.
// Out-of-range indices contribute nothing.
#include "common.hpp"

namespace aff {
namespace wg {

constexpr int THREADS = 256;
constexpr int NB = 8;
constexpr int ICB = 4;        // weighted_features: IC values per pass
constexpr int MERGE_KMAX = 128;

__device__ __forceinline__ int64_t load_index(const void *p, int is_i64, int64_t i) {
    return is_i64 ? static_cast<const int64_t *>(p)[i] : int64_t(static_cast<const int32_t *>(p)[i]);
}

struct WFArgs {
    const void *w; int w_dtype; int64_t w_sb, w_sn, w_sm, w_sic;
    const void *f; int64_t f_sb, f_sn;
    const void *idx; int idx_i64; int64_t i_sb, i_sn;
    void *out; int64_t o_sb, o_sn, o_sic;
    int B, Nout, Nsrc, M, C, IC;
};

// Vector path: C % 8 == 0 and 16-byte aligned rows.  LPR lanes per output
// row, each covering 8 channels per chunk; chunks stride LPR * 8.
template <typename T, int LPR>
__global__ __launch_bounds__(THREADS) void wfeat_vec_kernel(const WFArgs a) {
    using IO = ElemIO<T>;
    constexpr int ROWS = THREADS / LPR;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int sub = threadIdx.x % LPR;
    const int64_t row = (int64_t)bid * ROWS + threadIdx.x / LPR;
    if (row >= (int64_t)a.B * a.Nout) return;
    const int i = int(row % a.Nout), b = int(row / a.Nout);
    const T *F = static_cast<const T *>(a.f) + (int64_t)b * a.f_sb;
    const int64_t ibase = (int64_t)b * a.i_sb + (int64_t)i * a.i_sn;
    const int64_t wbase = (int64_t)b * a.w_sb + (int64_t)i * a.w_sn;
    T *O = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)i * a.o_sn;

    for (int c0 = sub * 8; c0 < a.C; c0 += LPR * 8) {
        for (int ic0 = 0; ic0 < a.IC; ic0 += ICB) {
            float acc[ICB][8];
#pragma unroll
            for (int t = 0; t < ICB; ++t)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[t][e] = 0.f;
            for (int m0 = 0; m0 < a.M; m0 += NB) {
                int64_t id[NB];
                bool ok[NB];
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    const int m = m0 + u;
                    id[u] = m < a.M ? load_index(a.idx, a.idx_i64, ibase + (int64_t)m * 1) : -1;
                    ok[u] = id[u] >= 0 && id[u] < a.Nsrc;
                }
                typename IO::raw8 fr[NB];
#pragma unroll
                for (int u = 0; u < NB; ++u) fr[u] = IO::load_raw(F + (ok[u] ? id[u] : 0) * a.f_sn + c0);
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    if (!ok[u]) continue;
                    float fv[8];
                    IO::cvt(fr[u], fv);
#pragma unroll
                    for (int t = 0; t < ICB; ++t) {
                        if (ic0 + t >= a.IC) break;
                        const float wv = load_any(a.w, a.w_dtype,
                                                  wbase + (int64_t)(m0 + u) * a.w_sm + (int64_t)(ic0 + t) * a.w_sic);
#pragma unroll
                        for (int e = 0; e < 8; ++e) acc[t][e] += wv * fv[e];
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < ICB; ++t)
                if (ic0 + t < a.IC) IO::store8(O + (int64_t)(ic0 + t) * a.o_sic + c0, acc[t]);
        }
    }
}

// IC = 4 with each row's weights packed [M][4] (the merge's layout): the four
// weights of a neighbour come as one vector load, and the next group's indices
// are loaded while the current group's rows are in flight.
template <typename TW>
__device__ __forceinline__ void load_w4(const TW *p, float (&o)[4]) {
    if constexpr (sizeof(TW) == 4) {
        const float4 v = *reinterpret_cast<const float4 *>(p);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    } else {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        const uint16_t h[4] = {uint16_t(v.x & 0xffffu), uint16_t(v.x >> 16), uint16_t(v.y & 0xffffu), uint16_t(v.y >> 16)};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (__is_same(TW, bf16_t)) o[i] = bf16_to_f32(h[i]);
            else o[i] = float(__builtin_bit_cast(_Float16, h[i]));
        }
    }
}

template <typename T, typename TW, bool IDX64, int LPR>
__global__ __launch_bounds__(THREADS) void wfeat4_kernel(const WFArgs a) {
    using IO = ElemIO<T>;
    constexpr int ROWS = THREADS / LPR;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int sub = threadIdx.x % LPR;
    const int64_t row = (int64_t)bid * ROWS + threadIdx.x / LPR;
    if (row >= (int64_t)a.B * a.Nout) return;
    const int i = int(row % a.Nout), b = int(row / a.Nout);
    const T *F = static_cast<const T *>(a.f) + (int64_t)b * a.f_sb;
    const int64_t ibase = (int64_t)b * a.i_sb + (int64_t)i * a.i_sn;
    const TW *W = static_cast<const TW *>(a.w) + (int64_t)b * a.w_sb + (int64_t)i * a.w_sn;
    T *O = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)i * a.o_sn;
    auto index = [&](int m) -> int {
        if (m >= a.M) return -1;
        const int64_t v = IDX64 ? static_cast<const int64_t *>(a.idx)[ibase + m]
                                : int64_t(static_cast<const int32_t *>(a.idx)[ibase + m]);
        return (v >= 0 && v < a.Nsrc) ? int(v) : -1;
    };
    for (int c0 = sub * 8; c0 < a.C; c0 += LPR * 8) {
        float acc[4][8];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[t][e] = 0.f;
        int id[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) id[u] = index(u);
        for (int m0 = 0; m0 < a.M; m0 += NB) {
            typename IO::raw8 fr[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) fr[u] = IO::load_raw(F + (int64_t)(id[u] >= 0 ? id[u] : 0) * a.f_sn + c0);
            float wv[NB][4];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                if (m0 + u < a.M) load_w4(W + (int64_t)(m0 + u) * 4, wv[u]);
                else wv[u][0] = wv[u][1] = wv[u][2] = wv[u][3] = 0.f;
            }
            int idn[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) idn[u] = index(m0 + NB + u);
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                if (id[u] < 0) continue;
                float fv[8];
                IO::cvt(fr[u], fv);
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[t][e] += wv[u][t] * fv[e];
            }
#pragma unroll
            for (int u = 0; u < NB; ++u) id[u] = idn[u];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) IO::store8(O + (int64_t)t * a.o_sic + c0, acc[t]);
    }
}

// Scalar path for any C / alignment: one lane per (row, channel).
template <typename T>
__global__ __launch_bounds__(THREADS) void wfeat_scalar_kernel(const WFArgs a) {
    const int64_t g = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.Nout * a.C;
    if (g >= total) return;
    const int c = int(g % a.C);
    const int64_t row = g / a.C;
    const int i = int(row % a.Nout), b = int(row / a.Nout);
    const int64_t ibase = (int64_t)b * a.i_sb + (int64_t)i * a.i_sn;
    const int64_t wbase = (int64_t)b * a.w_sb + (int64_t)i * a.w_sn;
    const T *F = static_cast<const T *>(a.f) + (int64_t)b * a.f_sb;
    T *O = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)i * a.o_sn;
    constexpr aff_dtype fdt = ElemIO<T>::code;
    for (int ic = 0; ic < a.IC; ++ic) {
        float acc = 0.f;
        for (int m = 0; m < a.M; ++m) {
            const int64_t id = load_index(a.idx, a.idx_i64, ibase + m);
            if (id < 0 || id >= a.Nsrc) continue;
            acc += load_any(a.w, a.w_dtype, wbase + (int64_t)m * a.w_sm + (int64_t)ic * a.w_sic) *
                   load_any(F, fdt, id * a.f_sn + c);
        }
        if constexpr (fdt == AFF_F32) reinterpret_cast<float *>(O)[(int64_t)ic * a.o_sic + c] = acc;
        else if constexpr (fdt == AFF_BF16) reinterpret_cast<uint16_t *>(O)[(int64_t)ic * a.o_sic + c] = f32_to_bf16(acc);
        else reinterpret_cast<_Float16 *>(O)[(int64_t)ic * a.o_sic + c] = _Float16(acc);
    }
}

// ----------------------------------------------------------- softmax merge --
struct MergeArgs {
    const float *qpos; int64_t q_sb, q_sn;   // [B, Nout, 2]
    const float *spos; int64_t s_sb, s_sn;   // [B, Nsrc, 2]
    const void *f; int64_t f_sb, f_sn;       // [B, Nsrc, C]
    const void *idx; int idx_i64; int64_t i_sb, i_sn;  // [B, Nout, K]
    float neg_inv_tau;
    void *out; int64_t o_sb, o_sn;           // [B, Nout, C]
    float *out_pos; int64_t op_sb, op_sn;    // [B, Nout, 2] or NULL
    float *out_w;                            // [B, Nout, K] contiguous or NULL
    int B, Nout, Nsrc, K, C;
};

template <int LPR>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (LPR >= 2) v = fmaxf(v, xor_lane<1>(v));
    if constexpr (LPR >= 4) v = fmaxf(v, xor_lane<2>(v));
    if constexpr (LPR >= 8) v = fmaxf(v, xor_lane<4>(v));
    if constexpr (LPR >= 16) v = fmaxf(v, xor_lane<8>(v));
    if constexpr (LPR >= 32) v = fmaxf(v, xor_lane<16>(v));
    if constexpr (LPR >= 64) v = fmaxf(v, xor_lane<32>(v));
    return v;
}

// d = sqrt(fl(fl(dx*dx) + fl(dy*dy))), the distance KNN ranked by.
__device__ __forceinline__ float euclid(float ax, float ay, float bx, float by) {
#pragma clang fp contract(off)
    const float dx = ax - bx, dy = ay - by;
    return sqrtf(dx * dx + dy * dy);
}

// Rows (merged points) per workgroup: at most 32, so the per-row weight and
// index staging (MERGE_KMAX * 8 bytes each) stays within 32 KB of LDS.
template <int LPR>
constexpr int merge_rows() { return (THREADS / LPR) < 32 ? (THREADS / LPR) : 32; }

template <typename T, int LPR>
__global__ __launch_bounds__(THREADS) void softmax_merge_kernel(const MergeArgs a) {
    using IO = ElemIO<T>;
    constexpr int ROWS = merge_rows<LPR>();
    __shared__ float s_w[ROWS][MERGE_KMAX];
    __shared__ int s_i[ROWS][MERGE_KMAX];
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int sub = threadIdx.x % LPR, slot = threadIdx.x / LPR;
    const int64_t row = (int64_t)bid * ROWS + slot;
    if (row >= (int64_t)a.B * a.Nout) return;   // whole groups leave together
    const int i = int(row % a.Nout), b = int(row / a.Nout);
    const float qx = a.qpos[(int64_t)b * a.q_sb + (int64_t)i * a.q_sn];
    const float qy = a.qpos[(int64_t)b * a.q_sb + (int64_t)i * a.q_sn + 1];
    const float *S = a.spos + (int64_t)b * a.s_sb;
    const int64_t ibase = (int64_t)b * a.i_sb + (int64_t)i * a.i_sn;

    // 1. logits -d/tau for this lane's neighbours, group max
    float mx = -INFINITY;
    for (int m = sub; m < a.K; m += LPR) {
        const int64_t id = load_index(a.idx, a.idx_i64, ibase + m);
        float lg = -INFINITY;
        if (id >= 0 && id < a.Nsrc) lg = euclid(qx, qy, S[id * a.s_sn], S[id * a.s_sn + 1]) * a.neg_inv_tau;
        s_w[slot][m] = lg;
        s_i[slot][m] = (id >= 0 && id < a.Nsrc) ? int(id) : -1;
        mx = fmaxf(mx, lg);
    }
    mx = group_max<LPR>(mx);
    // 2. exp, group sum, normalised weights, weighted coordinates
    float sum = 0.f;
    for (int m = sub; m < a.K; m += LPR) {
        const float e = __expf(s_w[slot][m] - mx);
        s_w[slot][m] = e;
        sum += e;
    }
    sum = group_sum<LPR>(sum);
    const float inv = 1.f / sum;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float px = 0.f, py = 0.f;
    for (int m = sub; m < a.K; m += LPR) {
        const float w = s_w[slot][m] * inv;
        s_w[slot][m] = w;
        const int id = s_i[slot][m];
        if (id >= 0) { px += w * S[(int64_t)id * a.s_sn]; py += w * S[(int64_t)id * a.s_sn + 1]; }
        if (a.out_w) a.out_w[row * a.K + m] = w;
    }
    px = group_sum<LPR>(px);
    py = group_sum<LPR>(py);
    if (a.out_pos && sub == 0) {
        a.out_pos[(int64_t)b * a.op_sb + (int64_t)i * a.op_sn] = px;
        a.out_pos[(int64_t)b * a.op_sb + (int64_t)i * a.op_sn + 1] = py;
    }
    // s_w / s_i of a group are written and read only by that group's lanes,
    // all in one wave: a wavefront-scope fence orders them (a workgroup
    // barrier is not usable after the early exit of tail groups).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 3. feature gather
    const T *F = static_cast<const T *>(a.f) + (int64_t)b * a.f_sb;
    T *O = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)i * a.o_sn;
    for (int c0 = sub * 8; c0 < a.C; c0 += LPR * 8) {
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        for (int m0 = 0; m0 < a.K; m0 += NB) {
            typename IO::raw8 fr[NB];
            float wv[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int m = m0 + u;
                const int id = m < a.K ? s_i[slot][m] : -1;
                wv[u] = id >= 0 ? s_w[slot][m] : 0.f;
                fr[u] = IO::load_raw(F + (int64_t)(id >= 0 ? id : 0) * a.f_sn + c0);
            }
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                float fv[8];
                IO::cvt(fr[u], fv);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] += wv[u] * fv[e];
            }
        }
        IO::store8(O + c0, acc);
    }
}

inline int lanes_for(int C) {
    int l = 1;
    while (l < 64 && l * 8 < C) l <<= 1;
    return l;
}

template <typename T>
aff_status launch_wfeat(const WFArgs &a, bool vec, hipStream_t s) {
    const int64_t rows = (int64_t)a.B * a.Nout;
    if (vec && a.IC == 4 && a.w_sic == 1 && a.w_sm == 4 &&
        (reinterpret_cast<uintptr_t>(a.w) & (a.w_dtype == AFF_F32 ? 15 : 7)) == 0 &&
        (a.w_sb * 4) % 16 == 0 && (a.w_sn * 4) % 16 == 0) {
        const int lpr = lanes_for(a.C);
        const int64_t blocks = (rows * lpr + THREADS - 1) / THREADS;
        auto go = [&](auto tw) {
            using TW = decltype(tw);
            switch (lpr) {
#define WF4_CASE(L)                                                                                             \
    case L:                                                                                                     \
        if (a.idx_i64) hipLaunchKernelGGL((wfeat4_kernel<T, TW, true, L>), dim3((unsigned)blocks), dim3(THREADS), 0, s, a); \
        else hipLaunchKernelGGL((wfeat4_kernel<T, TW, false, L>), dim3((unsigned)blocks), dim3(THREADS), 0, s, a);         \
        break;
                WF4_CASE(1) WF4_CASE(2) WF4_CASE(4) WF4_CASE(8) WF4_CASE(16) WF4_CASE(32) WF4_CASE(64)
#undef WF4_CASE
            }
        };
        if (a.w_dtype == AFF_F32) go(float{});
        else if (a.w_dtype == AFF_BF16) go(bf16_t{});
        else go(f16_t{});
    } else if (vec) {
        const int lpr = lanes_for(a.C);
        const int64_t blocks = (rows * lpr + THREADS - 1) / THREADS;
        switch (lpr) {
#define WF_CASE(L) case L: hipLaunchKernelGGL((wfeat_vec_kernel<T, L>), dim3((unsigned)blocks), dim3(THREADS), 0, s, a); break;
            WF_CASE(1) WF_CASE(2) WF_CASE(4) WF_CASE(8) WF_CASE(16) WF_CASE(32) WF_CASE(64)
#undef WF_CASE
        }
    } else {
        const int64_t blocks = (rows * a.C + THREADS - 1) / THREADS;
        hipLaunchKernelGGL(wfeat_scalar_kernel<T>, dim3((unsigned)blocks), dim3(THREADS), 0, s, a);
    }
    return check_launch("aff_weighted_features_fwd");
}

template <typename T>
aff_status launch_merge(const MergeArgs &a, hipStream_t s) {
    const int lpr = lanes_for(a.C);
    const int64_t rows = (int64_t)a.B * a.Nout;
    switch (lpr) {
#define MG_CASE(L) case L: { constexpr int R = merge_rows<L>(); \
        hipLaunchKernelGGL((softmax_merge_kernel<T, L>), dim3((unsigned)((rows + R - 1) / R)), dim3(R * L), 0, s, a); } break;
        MG_CASE(1) MG_CASE(2) MG_CASE(4) MG_CASE(8) MG_CASE(16) MG_CASE(32) MG_CASE(64)
#undef MG_CASE
    }
    return check_launch("aff_softmax_merge_fwd");
}

inline bool a16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace wg
}  // namespace aff

using namespace aff;

extern "C" aff_status aff_weighted_features_fwd(
    const void *weights, int w_dtype, int64_t w_sb, int64_t w_sn, int64_t w_sm, int64_t w_sic,
    const void *feat, int f_dtype, int64_t f_sb, int64_t f_sn,
    const void *nbhd_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn,
    int B, int Nout, int Nsrc, int M, int C, int IC,
    void *out, int64_t o_sb, int64_t o_sn, int64_t o_sic, aff_stream_t stream) {
    AFF_CHECK_ARG(B >= 0 && Nout >= 0 && Nsrc >= 0 && M >= 0 && C >= 0 && IC >= 1,
                  "aff_weighted_features_fwd: bad sizes B=%d Nout=%d Nsrc=%d M=%d C=%d IC=%d", B, Nout, Nsrc, M, C, IC);
    if (w_dtype < 0 || w_dtype > 2 || f_dtype < 0 || f_dtype > 2)
        return fail(AFF_ERR_UNSUPPORTED, "aff_weighted_features_fwd: dtype");
    if ((int64_t)B * Nout * C == 0) return AFF_OK;
    AFF_CHECK_ARG(feat && out && (M == 0 || (weights && nbhd_idx)), "aff_weighted_features_fwd: NULL pointer");
    wg::WFArgs a{weights, w_dtype, w_sb, w_sn, w_sm, w_sic, feat, f_sb, f_sn, nbhd_idx, idx_is_i64, i_sb, i_sn,
                 out, o_sb, o_sn, o_sic, B, Nout, Nsrc, M, C, IC};
    const int esz = f_dtype == AFF_F32 ? 4 : 2;
    bool vec = (C % 8 == 0) && wg::a16(feat) && wg::a16(out);
    for (int64_t s : {f_sb, f_sn, o_sb, o_sn, o_sic}) vec = vec && ((s * esz) % 16 == 0);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (f_dtype == AFF_F32) return wg::launch_wfeat<float>(a, vec, s);
    if (f_dtype == AFF_BF16) return wg::launch_wfeat<bf16_t>(a, vec, s);
    return wg::launch_wfeat<f16_t>(a, vec, s);
}

extern "C" aff_status aff_weighted_gather_fwd(
    const void *nbhd_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn,
    const void *weights, int w_dtype, int64_t w_sb, int64_t w_sn,
    const void *feat, int f_dtype, int64_t f_sb, int64_t f_sn,
    int B, int Nout, int Nsrc, int M, int C,
    void *out, int64_t o_sb, int64_t o_sn, aff_stream_t stream) {
    return aff_weighted_features_fwd(weights, w_dtype, w_sb, w_sn, 1, 0, feat, f_dtype, f_sb, f_sn, nbhd_idx,
                                     idx_is_i64, i_sb, i_sn, B, Nout, Nsrc, M, C, 1, out, o_sb, o_sn, 0, stream);
}

extern "C" aff_status aff_softmax_merge_fwd(
    const float *query_pos, int64_t q_sb, int64_t q_sn,
    const float *src_pos, int64_t s_sb, int64_t s_sn,
    const void *feat, int f_dtype, int64_t f_sb, int64_t f_sn,
    const void *nbhd_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn,
    int B, int Nout, int Nsrc, int K, int C, float tau,
    void *out, int64_t o_sb, int64_t o_sn,
    float *out_pos, int64_t op_sb, int64_t op_sn, float *out_weights, aff_stream_t stream) {
    AFF_CHECK_ARG(B >= 0 && Nout >= 0 && Nsrc >= 1 && K >= 1 && C >= 0,
                  "aff_softmax_merge_fwd: bad sizes B=%d Nout=%d Nsrc=%d K=%d C=%d", B, Nout, Nsrc, K, C);
    AFF_CHECK_ARG(K <= wg::MERGE_KMAX, "aff_softmax_merge_fwd: K=%d exceeds %d", K, wg::MERGE_KMAX);
    AFF_CHECK_ARG(tau > 0.f, "aff_softmax_merge_fwd: tau must be > 0");
    if (f_dtype < 0 || f_dtype > 2) return fail(AFF_ERR_UNSUPPORTED, "aff_softmax_merge_fwd: dtype");
    if ((int64_t)B * Nout == 0) return AFF_OK;
    AFF_CHECK_ARG(query_pos && src_pos && nbhd_idx && (C == 0 || (feat && out)), "aff_softmax_merge_fwd: NULL pointer");
    const int esz = f_dtype == AFF_F32 ? 4 : 2;
    bool vec = (C % 8 == 0) && (C == 0 || (wg::a16(feat) && wg::a16(out)));
    for (int64_t s : {f_sb, f_sn, o_sb, o_sn}) vec = vec && ((s * esz) % 16 == 0);
    if (!vec) return fail(AFF_ERR_UNSUPPORTED, "aff_softmax_merge_fwd: C must be a multiple of 8 with 16-byte aligned rows");
    wg::MergeArgs a{query_pos, q_sb, q_sn, src_pos, s_sb, s_sn, feat, f_sb, f_sn, nbhd_idx, idx_is_i64, i_sb, i_sn,
                    -1.f / tau, out, o_sb, o_sn, out_pos, op_sb, op_sn, out_weights, B, Nout, Nsrc, K, C};
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (f_dtype == AFF_F32) return wg::launch_merge<float>(a, s);
    if (f_dtype == AFF_BF16) return wg::launch_merge<bf16_t>(a, s);
    return wg::launch_merge<f16_t>(a, s);
}
