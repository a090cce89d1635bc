// Deformable attention over point clouds for gfx950.
//
// aff_deform_fwd: for every (b, q, h) and sample s = (level l, point p):
//   loc = query_pos[b, q] + offset[b, q, h, l, p]
//   exact K nearest points of loc among level l's points (ties -> lower index)
//   mode SHEPARD: w_j = softmax_j(-max(power, 1e-6) * (sqrt(d2_j) + 1e-6)), denominator + 1e-8
//                 (the live fused kernels, src/layers/kernels/fused_deform_attn.py:1188-1335, 842-1011)
//   mode IDW:     w_j = (1 / (d2_j^power + 1e-10)) / (sum + 1e-12)
//                 (inverse_distance_weighting, src/utils/geometry.py:40-53, on squared distances)
//   out[b, q, h, :] = sum_s attn[b, q, h, s] * sum_j w_j * values[b, level_row(l, j), h, :]
// Phase A (one lane per sample) finds the neighbours on the level's cell grid
// (grid2d.hpp) and stages (row, attn * w) pairs in LDS; phase B gathers the
// value rows (8 channels per lane, 16-byte loads) and reduces in fp32.  The
// neighbour indices never go to HBM unless the caller asks for them.
//
// aff_deform_sample_fwd: the same weights from given neighbour indices
//   (fused_deformable_attention, fused_deform_attn.py:79-231, 503-571: sqrt(d2) + 1e-6;
//    mssample, mssample.py:17-125, 300-342: sqrt(d2 + 1e-6)); optional gather.
//
// aff_msdetrpc_fwd: out[b,n,:] = sum_m sum_k attn[b,n,m] * w[b,n,m,k] * val[b, idx[b,n,m,k], :]
//   (msdetrpc.py:25-109).
#include "grid2d.hpp"

namespace aff {
namespace deform {

using namespace grid;

constexpr int THREADS = 256;
constexpr int KMAX = 8;    // neighbours per sample
constexpr int CAP = 16;    // per-lane candidate list of the neighbour search
constexpr int NB = 8;

__device__ __forceinline__ int64_t load_index(const void *p, int is_i64, int64_t i) {
    return is_i64 ? static_cast<const int64_t *>(p)[i] : int64_t(static_cast<const int32_t *>(p)[i]);
}

struct KArgs {
    aff_deform_args a;
    Segs segs;
    WsLayout wl;
    const void *ws;
};

// SPR: lanes per (b, q, h) row = next power of two >= L * P.
template <typename T, int SPR>
__global__ __launch_bounds__(THREADS) void deform_fwd_kernel(const KArgs ka) {
    using IO = ElemIO<T>;
    constexpr int R = THREADS / SPR;             // rows per workgroup
    __shared__ uint64_t s_list[CAP * THREADS];   // neighbour search, one column per lane
    __shared__ int s_row[R][SPR * KMAX];
    __shared__ float s_w[R][SPR * KMAX];
    __shared__ float s_red[THREADS * 8];

    const aff_deform_args &a = ka.a;
    const int tid = threadIdx.x;
    const int r = tid / SPR, t = tid % SPR;
    const int S = a.L * a.P, K = a.K;
    const int64_t total = (int64_t)a.B * a.Nq * a.H;
    const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * R + r;
    const bool active = row < total;
    const int h = active ? int(row % a.H) : 0;
    const int64_t bq = active ? row / a.H : 0;
    const int q = int(bq % a.Nq), b = int(bq / a.Nq);

    // ---- phase A: one lane per sample
    // pairs of sample t occupy slots [t * K, t * K + K)
    for (int j = 0; j < KMAX; ++j) {
        s_row[r][t * KMAX + j] = -1;
        s_w[r][t * KMAX + j] = 0.f;
    }
    __syncthreads();
    if (active && t < S) {
        const int l = t / a.P;
        const float qx = a.query_pos[(int64_t)b * a.qp_sb + (int64_t)q * a.qp_sn];
        const float qy = a.query_pos[(int64_t)b * a.qp_sb + (int64_t)q * a.qp_sn + 1];
        const int64_t ob = (int64_t)b * a.off_sb + (int64_t)q * a.off_sn + (int64_t)h * a.off_sh + (int64_t)t * 2;
        const float sx = qx + load_any(a.offsets, a.off_dtype, ob);
        const float sy = qy + load_any(a.offsets, a.off_dtype, ob + 1);
        const float aw =
            load_any(a.attn, a.attn_dtype, (int64_t)b * a.at_sb + (int64_t)q * a.at_sn + (int64_t)h * a.at_sh + t);
        const float pw = *a.power;
        const SegView g = seg_view(ka.ws, ka.wl, ka.segs, b, l);
        const int keff = min(K, g.n);
        uint64_t keys[CAP];
        if (keff > 0) {
            knn_select<CAP>(g, sx, sy, keff, s_list + tid, THREADS, keys);
        } else {
#pragma unroll
            for (int j = 0; j < CAP; ++j) keys[j] = ~0ull;
        }
        float wj[KMAX];
        float wsum = 0.f;
        if (a.mode == AFF_DEFORM_SHEPARD) {
            const float p = fmaxf(pw, 1e-6f);
            float lg[KMAX], mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < KMAX; ++j) {
                lg[j] = -INFINITY;
                if (j < keff) lg[j] = -p * (sqrtf(key_d2(keys[j])) + 1e-6f);
                mx = fmaxf(mx, lg[j]);
            }
#pragma unroll
            for (int j = 0; j < KMAX; ++j) {
                wj[j] = j < keff ? __expf(lg[j] - mx) : 0.f;
                wsum += wj[j];
            }
            wsum += 1e-8f;
        } else {
#pragma unroll
            for (int j = 0; j < KMAX; ++j) {
                wj[j] = j < keff ? 1.f / (powf(key_d2(keys[j]), pw) + 1e-10f) : 0.f;
                wsum += wj[j];
            }
            wsum += 1e-12f;
        }
        const float inv = 1.f / wsum;
        const int64_t kb = ((row * a.L * a.P) + t) * K;   // [B, Nq, H, L, P, K]
        const int lstart = ka.segs.start[l];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            if (j < keff) {
                s_row[r][t * K + j] = key_index(keys[j]);
                s_w[r][t * K + j] = aw * wj[j] * inv;
            }
            if (j < K) {
                if (a.knn_idx) a.knn_idx[kb + j] = j < keff ? key_index(keys[j]) - lstart : -1;
                if (a.knn_d2) a.knn_d2[kb + j] = j < keff ? key_d2(keys[j]) : INFINITY;
            }
        }
    }
    __syncthreads();

    // ---- phase B: value gather.  Lane t of a row: channel chunk cc = t % CG,
    // pair subset sg = t / CG (pairs sg, sg + NSG, ...), then sum subsets.
    const int C = a.C, CG = C / 8;
    const int NSG = SPR >= CG ? SPR / CG : 1;
    const int npair = S * K;
    const T *V = static_cast<const T *>(a.values) + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh;
    T *O = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)q * a.o_sn + (int64_t)h * a.o_sh;
    if (SPR >= CG) {
        const int cc = t % CG, sg = t / CG;
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        if (active && sg < NSG) {
            for (int j0 = sg; j0 < npair; j0 += NSG * NB) {
                typename IO::raw8 fr[NB];
                float wv[NB];
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    const int j = j0 + u * NSG;
                    const int rr = j < npair ? s_row[r][j] : -1;
                    wv[u] = rr >= 0 ? s_w[r][j] : 0.f;
                    fr[u] = IO::load_raw(V + (int64_t)(rr >= 0 ? rr : 0) * a.v_sn + cc * 8);
                }
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    float fv[8];
                    IO::cvt(fr[u], fv);
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[e] += wv[u] * fv[e];
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) s_red[tid * 8 + e] = acc[e];
        __syncthreads();
        if (active && sg == 0) {
            for (int o = 1; o < NSG; ++o) {
                const int src = (r * SPR + o * CG + cc) * 8;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] += s_red[src + e];
            }
            IO::store8(O + cc * 8, acc);
        }
    } else if (active) {
        for (int cc = t; cc < CG; cc += SPR) {
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = 0.f;
            for (int j0 = 0; j0 < npair; j0 += NB) {
                typename IO::raw8 fr[NB];
                float wv[NB];
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    const int j = j0 + u;
                    const int rr = j < npair ? s_row[r][j] : -1;
                    wv[u] = rr >= 0 ? s_w[r][j] : 0.f;
                    fr[u] = IO::load_raw(V + (int64_t)(rr >= 0 ? rr : 0) * a.v_sn + cc * 8);
                }
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    float fv[8];
                    IO::cvt(fr[u], fv);
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[e] += wv[u] * fv[e];
                }
            }
            IO::store8(O + cc * 8, acc);
        }
    }
}

// ------------------------------------------------ given neighbour indices --
struct SArgs {
    int eps_mode;      // 0: sqrt(d2) + 1e-6 (fused_deformable_attention), 1: sqrt(d2 + 1e-6) (mssample)
    int B, N, Nkv, K, D, C;
    const float *loc; int64_t l_sb, l_sn;
    const float *kv; int64_t k_sb, k_sn;
    const void *idx; int idx_i64; int64_t i_sb, i_sn;
    const float *power;
    const void *attn; int attn_dtype; int64_t a_sb, a_sn;
    const void *values; int64_t v_sb, v_sn;
    void *out; int64_t o_sb, o_sn;
    void *weights; int w_dtype; int64_t w_sb, w_sn;
};

constexpr int SK_MAX = 64;

// One lane group of LPR lanes per sampling location.
template <typename T, int LPR>
__global__ __launch_bounds__(THREADS) void deform_sample_kernel(const SArgs a) {
    using IO = ElemIO<T>;
    constexpr int R = THREADS / LPR;
    __shared__ float s_w[R][SK_MAX];
    __shared__ int s_i[R][SK_MAX];
    const int tid = threadIdx.x, r = tid / LPR, t = tid % LPR;
    const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * R + r;
    if (row >= (int64_t)a.B * a.N) return;   // whole groups leave together
    const int n = int(row % a.N), b = int(row / a.N);
    const float *Lc = a.loc + (int64_t)b * a.l_sb + (int64_t)n * a.l_sn;
    const float *KV = a.kv + (int64_t)b * a.k_sb;
    const int64_t ib = (int64_t)b * a.i_sb + (int64_t)n * a.i_sn;
    const float p = fmaxf(*a.power, 1e-6f);
    float mx = -INFINITY;
    for (int j = t; j < a.K; j += LPR) {
        const int64_t id = load_index(a.idx, a.idx_i64, ib + j);
        float lg = -INFINITY;
        if (id >= 0 && id < a.Nkv) {
            float d2 = 0.f;
            for (int d = 0; d < a.D; ++d) {
                const float df = Lc[d] - KV[id * a.k_sn + d];
                d2 += df * df;
            }
            const float dist = a.eps_mode == 0 ? sqrtf(d2) + 1e-6f : sqrtf(d2 + 1e-6f);
            lg = -p * dist;
        }
        s_w[r][j] = lg;
        s_i[r][j] = (id >= 0 && id < a.Nkv) ? int(id) : -1;
        mx = fmaxf(mx, lg);
    }
    float m2 = mx;
    if constexpr (LPR >= 2) m2 = fmaxf(m2, xor_lane<1>(m2));
    if constexpr (LPR >= 4) m2 = fmaxf(m2, xor_lane<2>(m2));
    if constexpr (LPR >= 8) m2 = fmaxf(m2, xor_lane<4>(m2));
    if constexpr (LPR >= 16) m2 = fmaxf(m2, xor_lane<8>(m2));
    if constexpr (LPR >= 32) m2 = fmaxf(m2, xor_lane<16>(m2));
    if constexpr (LPR >= 64) m2 = fmaxf(m2, xor_lane<32>(m2));
    float sum = 0.f;
    for (int j = t; j < a.K; j += LPR) {
        const float e = s_i[r][j] >= 0 ? __expf(s_w[r][j] - m2) : 0.f;
        s_w[r][j] = e;
        sum += e;
    }
    sum = group_sum<LPR>(sum);
    const float inv = 1.f / (sum + 1e-8f);
    const float aw = a.attn ? load_any(a.attn, a.attn_dtype, (int64_t)b * a.a_sb + (int64_t)n * a.a_sn) : 1.f;
    for (int j = t; j < a.K; j += LPR) {
        const float w = s_w[r][j] * inv;
        s_w[r][j] = w * aw;
        if (a.weights) {
            const int64_t o = (int64_t)b * a.w_sb + (int64_t)n * a.w_sn + j;
            if (a.w_dtype == AFF_F32) static_cast<float *>(a.weights)[o] = w;
            else if (a.w_dtype == AFF_BF16) static_cast<uint16_t *>(a.weights)[o] = f32_to_bf16(w);
            else static_cast<_Float16 *>(a.weights)[o] = _Float16(w);
        }
    }
    if (!a.out) return;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const T *V = static_cast<const T *>(a.values) + (int64_t)b * a.v_sb;
    T *O = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)n * a.o_sn;
    for (int c0 = t * 8; c0 < a.C; c0 += LPR * 8) {
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        for (int j0 = 0; j0 < a.K; j0 += NB) {
            typename IO::raw8 fr[NB];
            float wv[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int j = j0 + u;
                const int id = j < a.K ? s_i[r][j] : -1;
                wv[u] = id >= 0 ? s_w[r][j] : 0.f;
                fr[u] = IO::load_raw(V + (int64_t)(id >= 0 ? id : 0) * a.v_sn + c0);
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

// ------------------------------------------------------------- MSDETRPC --
struct MArgs {
    const void *idx; int idx_i64; int64_t i_sb, i_sn, i_sm;   // [B, N, M, K], unit stride on K
    const void *w; int w_dtype; int64_t w_sb, w_sn, w_sm;     // [B, N, M, K], unit stride on K
    const void *attn; int a_dtype; int64_t a_sb, a_sn;        // [B, N, M], unit stride on M
    const void *val; int64_t v_sb, v_sn;                      // [B, Nval, C]
    void *out; int64_t o_sb, o_sn;                            // [B, N, C]
    int B, N, M, K, Nval, C;
};

template <typename T, int LPR>
__global__ __launch_bounds__(THREADS) void msdetrpc_kernel(const MArgs a) {
    using IO = ElemIO<T>;
    constexpr int R = THREADS / LPR;
    const int r = threadIdx.x / LPR, t = threadIdx.x % LPR;
    const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * R + r;
    if (row >= (int64_t)a.B * a.N) return;
    const int n = int(row % a.N), b = int(row / a.N);
    const T *V = static_cast<const T *>(a.val) + (int64_t)b * a.v_sb;
    T *O = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)n * a.o_sn;
    const int np = a.M * a.K;
    for (int c0 = t * 8; c0 < a.C; c0 += LPR * 8) {
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        for (int j0 = 0; j0 < np; j0 += NB) {
            typename IO::raw8 fr[NB];
            float wv[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int j = j0 + u;
                int64_t id = -1;
                wv[u] = 0.f;
                if (j < np) {
                    const int m = j / a.K, kk = j % a.K;
                    id = load_index(a.idx, a.idx_i64, (int64_t)b * a.i_sb + (int64_t)n * a.i_sn + (int64_t)m * a.i_sm + kk);
                    if (id >= 0 && id < a.Nval)
                        wv[u] = load_any(a.attn, a.a_dtype, (int64_t)b * a.a_sb + (int64_t)n * a.a_sn + m) *
                                load_any(a.w, a.w_dtype, (int64_t)b * a.w_sb + (int64_t)n * a.w_sn + (int64_t)m * a.w_sm + kk);
                    else
                        id = -1;
                }
                fr[u] = IO::load_raw(V + (id >= 0 ? id : 0) * a.v_sn + c0);
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

inline int pow2_at_least(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}
inline int lanes_for(int C) {
    int l = 1;
    while (l < 64 && l * 8 < C) l <<= 1;
    return l;
}
inline bool a16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename T>
aff_status launch_deform(const KArgs &ka, int spr, hipStream_t s) {
    const int64_t rows = (int64_t)ka.a.B * ka.a.Nq * ka.a.H;
    const int64_t blocks = (rows * spr + THREADS - 1) / THREADS;
    switch (spr) {
#define DF_CASE(S) case S: hipLaunchKernelGGL((deform_fwd_kernel<T, S>), dim3((unsigned)blocks), dim3(THREADS), 0, s, ka); break;
        DF_CASE(1) DF_CASE(2) DF_CASE(4) DF_CASE(8) DF_CASE(16) DF_CASE(32)
#undef DF_CASE
        default: return fail(AFF_ERR_UNSUPPORTED, "aff_deform_fwd: L*P=%d exceeds 32", spr);
    }
    return check_launch("aff_deform_fwd");
}

template <typename T>
aff_status launch_sample(const SArgs &sa, hipStream_t s) {
    const int lpr = lanes_for(sa.out ? sa.C : 8);
    const int64_t rows = (int64_t)sa.B * sa.N;
    const int64_t blocks = (rows * lpr + THREADS - 1) / THREADS;
    switch (lpr) {
#define SM_CASE(L) case L: hipLaunchKernelGGL((deform_sample_kernel<T, L>), dim3((unsigned)blocks), dim3(THREADS), 0, s, sa); break;
        SM_CASE(1) SM_CASE(2) SM_CASE(4) SM_CASE(8) SM_CASE(16) SM_CASE(32) SM_CASE(64)
#undef SM_CASE
    }
    return check_launch("aff_deform_sample_fwd");
}

template <typename T>
aff_status launch_msdetrpc(const MArgs &ma, hipStream_t s) {
    const int lpr = lanes_for(ma.C);
    const int64_t rows = (int64_t)ma.B * ma.N;
    const int64_t blocks = (rows * lpr + THREADS - 1) / THREADS;
    switch (lpr) {
#define MS_CASE(L) case L: hipLaunchKernelGGL((msdetrpc_kernel<T, L>), dim3((unsigned)blocks), dim3(THREADS), 0, s, ma); break;
        MS_CASE(1) MS_CASE(2) MS_CASE(4) MS_CASE(8) MS_CASE(16) MS_CASE(32) MS_CASE(64)
#undef MS_CASE
    }
    return check_launch("aff_msdetrpc_fwd");
}

aff_status check_common(const aff_deform_args &a, Segs &segs) {
    AFF_CHECK_ARG(a.mode == AFF_DEFORM_SHEPARD || a.mode == AFF_DEFORM_IDW, "aff_deform_fwd: mode %d", a.mode);
    AFF_CHECK_ARG(a.B >= 0 && a.Nq >= 0 && a.H >= 1 && a.P >= 1 && a.C >= 0,
                  "aff_deform_fwd: bad sizes B=%d Nq=%d H=%d P=%d C=%d", a.B, a.Nq, a.H, a.P, a.C);
    AFF_CHECK_ARG(a.L >= 1 && a.L <= AFF_DEFORM_MAX_LEVELS, "aff_deform_fwd: L=%d outside [1, %d]", a.L,
                  AFF_DEFORM_MAX_LEVELS);
    AFF_CHECK_ARG(a.K >= 1 && a.K <= KMAX, "aff_deform_fwd: K=%d outside [1, %d]", a.K, KMAX);
    AFF_CHECK_ARG(a.level_start[0] == 0, "aff_deform_fwd: level_start[0] must be 0");
    int n[AFF_DEFORM_MAX_LEVELS];
    for (int l = 0; l < a.L; ++l) {
        n[l] = a.level_start[l + 1] - a.level_start[l];
        AFF_CHECK_ARG(n[l] >= 0, "aff_deform_fwd: level_start must be non-decreasing");
    }
    segs = make_segs(a.L, n);
    return AFF_OK;
}

}  // namespace deform
}  // namespace aff

using namespace aff;

extern "C" size_t aff_deform_workspace_bytes(const aff_deform_args *args) {
    if (!args || args->L < 1 || args->L > AFF_DEFORM_MAX_LEVELS || args->B <= 0) return 0;
    grid::Segs segs;
    if (deform::check_common(*args, segs) != AFF_OK) return 0;
    return grid::ws_layout(args->B, segs).total;
}

extern "C" aff_status aff_deform_fwd(const aff_deform_args *args, void *ws, size_t ws_bytes, aff_stream_t stream) {
    AFF_CHECK_ARG(args != nullptr, "aff_deform_fwd: NULL args");
    const aff_deform_args &a = *args;
    grid::Segs segs;
    aff_status st = deform::check_common(a, segs);
    if (st != AFF_OK) return st;
    if (a.dtype != AFF_F32 && a.dtype != AFF_F16 && a.dtype != AFF_BF16)
        return fail(AFF_ERR_UNSUPPORTED, "aff_deform_fwd: dtype %d", a.dtype);
    AFF_CHECK_ARG(a.C % 8 == 0, "aff_deform_fwd: channels per head C=%d must be a multiple of 8", a.C);
    if ((int64_t)a.B * a.Nq * a.H == 0) return AFF_OK;
    AFF_CHECK_ARG(a.query_pos && a.kv_pos && a.offsets && a.attn && a.values && a.out && a.power,
                  "aff_deform_fwd: NULL pointer");
    AFF_CHECK_ARG(a.off_dtype >= 0 && a.off_dtype <= 2 && a.attn_dtype >= 0 && a.attn_dtype <= 2,
                  "aff_deform_fwd: offset/attention dtype");
    const int esz = a.dtype == AFF_F32 ? 4 : 2;
    for (int64_t s : {a.v_sb, a.v_sn, a.v_sh, a.o_sb, a.o_sn, a.o_sh})
        AFF_CHECK_ARG((s * esz) % 16 == 0, "aff_deform_fwd: value/output strides must keep 16-byte rows");
    AFF_CHECK_ARG(deform::a16(a.values) && deform::a16(a.out), "aff_deform_fwd: values/out must be 16-byte aligned");
    const int spr = deform::pow2_at_least(a.L * a.P);
    if (spr > 32) return fail(AFF_ERR_UNSUPPORTED, "aff_deform_fwd: L*P=%d exceeds 32 samples per head", a.L * a.P);
    const grid::WsLayout wl = grid::ws_layout(a.B, segs);
    if (!ws || ws_bytes < wl.total)
        return fail(AFF_ERR_WORKSPACE, "aff_deform_fwd: workspace of %zu bytes needed, got %zu", wl.total, ws_bytes);
    AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(ws) & 255) == 0, "aff_deform_fwd: workspace must be 256-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    st = grid::launch_build(a.kv_pos, a.kp_sb, a.kp_sn, a.B, segs, ws, s);
    if (st != AFF_OK) return st;
    deform::KArgs ka{a, segs, wl, ws};
    if (a.dtype == AFF_F32) return deform::launch_deform<float>(ka, spr, s);
    if (a.dtype == AFF_BF16) return deform::launch_deform<bf16_t>(ka, spr, s);
    return deform::launch_deform<f16_t>(ka, spr, s);
}

extern "C" aff_status aff_deform_sample_fwd(int eps_mode, const float *sampling_locs, int64_t l_sb, int64_t l_sn,
                                            const float *kv_pos, int64_t k_sb, int64_t k_sn,
                                            const void *nb_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn,
                                            const float *power, int B, int N, int Nkv, int K, int D,
                                            const void *attn, int attn_dtype, int64_t a_sb, int64_t a_sn,
                                            const void *values, int dtype, int64_t v_sb, int64_t v_sn, int C,
                                            void *out, int64_t o_sb, int64_t o_sn,
                                            void *weights, int w_dtype, int64_t w_sb, int64_t w_sn,
                                            aff_stream_t stream) {
    AFF_CHECK_ARG(eps_mode == 0 || eps_mode == 1, "aff_deform_sample_fwd: eps_mode %d", eps_mode);
    AFF_CHECK_ARG(B >= 0 && N >= 0 && Nkv >= 0 && K >= 1 && K <= deform::SK_MAX && D >= 1 && D <= 4,
                  "aff_deform_sample_fwd: bad sizes B=%d N=%d Nkv=%d K=%d D=%d", B, N, Nkv, K, D);
    AFF_CHECK_ARG(out || weights, "aff_deform_sample_fwd: nothing to compute (out and weights NULL)");
    if ((int64_t)B * N == 0) return AFF_OK;
    AFF_CHECK_ARG(sampling_locs && kv_pos && nb_idx && power, "aff_deform_sample_fwd: NULL pointer");
    if (out) {
        AFF_CHECK_ARG(values && C >= 0 && C % 8 == 0, "aff_deform_sample_fwd: values with C %% 8 == 0 required");
        if (dtype < 0 || dtype > 2) return fail(AFF_ERR_UNSUPPORTED, "aff_deform_sample_fwd: dtype");
        const int esz = dtype == AFF_F32 ? 4 : 2;
        for (int64_t s : {v_sb, v_sn, o_sb, o_sn})
            AFF_CHECK_ARG((s * esz) % 16 == 0, "aff_deform_sample_fwd: value/output strides must keep 16-byte rows");
        AFF_CHECK_ARG(deform::a16(values) && deform::a16(out), "aff_deform_sample_fwd: values/out alignment");
    } else {
        dtype = AFF_F32;
    }
    if (weights) AFF_CHECK_ARG(w_dtype >= 0 && w_dtype <= 2, "aff_deform_sample_fwd: weights dtype");
    deform::SArgs sa{eps_mode, B, N, Nkv, K, D, C, sampling_locs, l_sb, l_sn, kv_pos, k_sb, k_sn,
                     nb_idx, idx_is_i64, i_sb, i_sn, power, attn, attn_dtype, a_sb, a_sn,
                     values, v_sb, v_sn, out, o_sb, o_sn, weights, w_dtype, w_sb, w_sn};
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == AFF_F32) return deform::launch_sample<float>(sa, s);
    if (dtype == AFF_BF16) return deform::launch_sample<bf16_t>(sa, s);
    return deform::launch_sample<f16_t>(sa, s);
}

extern "C" aff_status aff_msdetrpc_fwd(const void *nn_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn, int64_t i_sm,
                                       const void *nn_weight, int w_dtype, int64_t w_sb, int64_t w_sn, int64_t w_sm,
                                       const void *attn, int a_dtype, int64_t a_sb, int64_t a_sn,
                                       const void *val, int dtype, int64_t v_sb, int64_t v_sn,
                                       int B, int N, int M, int K, int Nval, int C,
                                       void *out, int64_t o_sb, int64_t o_sn, aff_stream_t stream) {
    AFF_CHECK_ARG(B >= 0 && N >= 0 && M >= 0 && K >= 0 && Nval >= 0 && C >= 0,
                  "aff_msdetrpc_fwd: bad sizes B=%d N=%d M=%d K=%d Nval=%d C=%d", B, N, M, K, Nval, C);
    if (dtype < 0 || dtype > 2 || w_dtype < 0 || w_dtype > 2 || a_dtype < 0 || a_dtype > 2)
        return fail(AFF_ERR_UNSUPPORTED, "aff_msdetrpc_fwd: dtype");
    AFF_CHECK_ARG(C % 8 == 0, "aff_msdetrpc_fwd: C=%d must be a multiple of 8", C);
    if ((int64_t)B * N * C == 0) return AFF_OK;
    AFF_CHECK_ARG(val && out && (M * K == 0 || (nn_idx && nn_weight && attn)), "aff_msdetrpc_fwd: NULL pointer");
    const int esz = dtype == AFF_F32 ? 4 : 2;
    for (int64_t s : {v_sb, v_sn, o_sb, o_sn})
        AFF_CHECK_ARG((s * esz) % 16 == 0, "aff_msdetrpc_fwd: value/output strides must keep 16-byte rows");
    AFF_CHECK_ARG(deform::a16(val) && deform::a16(out), "aff_msdetrpc_fwd: val/out must be 16-byte aligned");
    deform::MArgs ma{nn_idx, idx_is_i64, i_sb, i_sn, i_sm, nn_weight, w_dtype, w_sb, w_sn, w_sm,
                     attn, a_dtype, a_sb, a_sn, val, v_sb, v_sn, out, o_sb, o_sn, B, N, M, K, Nval, C};
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == AFF_F32) return deform::launch_msdetrpc<float>(ma, s);
    if (dtype == AFF_BF16) return deform::launch_msdetrpc<bf16_t>(ma, s);
    return deform::launch_msdetrpc<f16_t>(ma, s);
}
