// Backward of the deformable gathers for gfx950 (aff_deform_bwd).
//
// Three passes, none with float atomics:
//  1. rows_kernel: one group of G lanes per row r = (b, q, h) (8 channels of
//     dout per lane and chunk).  Per sample it recomputes the forward's
//     weights from the positions, takes <dout, value row> for each neighbour
//     (a G-lane reduction), and writes d_attn / d_weights / d_loc and the
//     row's d_power term directly.  Every pair (r, s, j) leaves its d_values
//     coefficient attn * w_j, its d_kv_pos term and a bucket key (the value
//     row (b, row, h) it adds into) in the workspace.
//  2. The pairs are bucketed by a stable radix sort (bucket.hpp), so each
//     value row lists the pairs that add into it in pair order.
//  3. dvalues_kernel sums coef * dout over each bucket (G lanes per value
//     row, 8 channels each); dkv_kernel sums the position terms of the H
//     buckets of each point; sum_kernel folds the per-row d_power terms in a
//     fixed tree.  Hence the results do not depend on scheduling.
// The chain rule (reference fused_deform_attn.py:2014-2186, 253-500,
// mssample.py:142-298, msdetrpc.py:133-300) is restated in include/affmae.h.
#include "bucket.hpp"

#include <math.h>

namespace aff {
namespace dbwd {

constexpr int THREADS = 256;
constexpr int KMAX = 16;     // neighbours per sample
constexpr int DMAX = 4;      // position dimensions
constexpr int NCHMAX = 4;    // chunks of 8 channels per lane: C <= 8 * 64 * NCHMAX
constexpr int SUM_CHUNKS = 256;

__device__ __forceinline__ int64_t load_idx(const void *p, int is_i64, int64_t i) {
    return is_i64 ? static_cast<const int64_t *>(p)[i] : int64_t(static_cast<const int32_t *>(p)[i]);
}

struct Work {
    unsigned *keys;   // [pairs]: bucket (b * Nkv + row) * H + h, or nkeys for none
    int *ids;         // [pairs]: pair id
    float *coef;      // [pairs]: attn * w (d_values)
    float *gkv;       // [pairs * D]: d_kv_pos term
    float *dpow_row;  // [rows]
    bool keyed;       // keys / ids / coef / gkv wanted
};

__device__ __forceinline__ bool is_dist_mode(int m) { return m != AFF_DEFORM_BWD_GIVEN; }

// d2 ^ e for the IDW forward's exponents: a product chain for 0..4, exp2(e log2 d2) otherwise.
__device__ __forceinline__ float pow_like_fwd(float d2, float e, int ie) {
    if (ie == 0) return 1.f;
    if (ie == 1) return d2;
    if (ie == 2) return d2 * d2;
    if (ie == 3) return d2 * d2 * d2;
    if (ie == 4) return (d2 * d2) * (d2 * d2);
    return __builtin_amdgcn_exp2f(e * __builtin_amdgcn_logf(d2));
}

__device__ __forceinline__ int int_exponent(float e) {
    return (e == 0.f || e == 1.f || e == 2.f || e == 3.f || e == 4.f) ? int(e) : -1;
}

template <typename T, int G, int NCH>
__global__ __launch_bounds__(THREADS) void rows_kernel(const aff_deform_bwd_args a, const Work w) {
    using IO = ElemIO<T>;
    constexpr int RPB = THREADS / G;
    const int sub = threadIdx.x % G;
    const int64_t r = (int64_t)blockIdx.x * RPB + threadIdx.x / G;
    const int64_t R = (int64_t)a.B * a.Q * a.H;
    if (r >= R) return;  // whole groups leave together
    const int h = int(r % a.H);
    const int64_t bq = r / a.H;
    const int q = int(bq % a.Q), b = int(bq / a.Q);
    const int S = a.S, K = a.K, D = a.D;
    const bool dist_mode = is_dist_mode(a.mode);

    // dout chunk(s) of this lane
    float dof[NCH > 0 ? NCH : 1][8];
    const T *dout = static_cast<const T *>(a.dout) + (int64_t)b * a.do_sb + (int64_t)q * a.do_sn + (int64_t)h * a.do_sh;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c0 = 8 * (sub + G * k);
        if (c0 < a.C) IO::load8(dout + c0, dof[k]);
        else
#pragma unroll
            for (int i = 0; i < 8; ++i) dof[k][i] = 0.f;
    }
    const T *V = a.values ? static_cast<const T *>(a.values) + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh : nullptr;
    const float *KV = a.kv_pos ? a.kv_pos + (int64_t)b * a.kp_sb : nullptr;
    const float praw = a.power ? *a.power : 0.f;
    const float pw = fmaxf(praw, 1e-6f);
    const int ie = int_exponent(praw);
    float lb[DMAX] = {0.f, 0.f, 0.f, 0.f};
    if (a.loc) {
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < D) lb[d] = a.loc[(int64_t)b * a.loc_sb + (int64_t)q * a.loc_sn + d];
    }
    const int64_t ib = (int64_t)b * a.i_sb + (int64_t)q * a.i_sn + (int64_t)h * a.i_sh;
    const int64_t ob = (int64_t)b * a.off_sb + (int64_t)q * a.off_sn + (int64_t)h * a.off_sh;
    const int64_t atb = (int64_t)b * a.at_sb + (int64_t)q * a.at_sn + (int64_t)h * a.at_sh;
    const int64_t wb = (int64_t)b * a.w_sb + (int64_t)q * a.w_sn + (int64_t)h * a.w_sh;
    const int64_t dwb = (int64_t)b * a.dwi_sb + (int64_t)q * a.dwi_sn + (int64_t)h * a.dwi_sh;
    const unsigned nkeys = unsigned((int64_t)a.B * a.Nkv * a.H);
    float dpow = 0.f;

    for (int s = 0; s < S; ++s) {
        const int l = s / a.P;
        const int lo = a.level_start[l], hi = a.level_start[l + 1];
        float loc[DMAX];
#pragma unroll
        for (int d = 0; d < DMAX; ++d) {
            loc[d] = lb[d];
            if (d < D && a.offsets) loc[d] = lb[d] + load_any(a.offsets, a.off_dtype, ob + (int64_t)s * D + d);
        }
        const float aw = a.attn ? load_any(a.attn, a.attn_dtype, atb + s) : 1.f;
        int row[KMAX];
        float d2[KMAX], wj[KMAX], gj[KMAX];
        // neighbours, distances, forward weights
        float mx = -INFINITY, usum = 0.f;
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            row[j] = -1;
            d2[j] = 0.f;
            wj[j] = 0.f;
            if (j >= K) continue;
            const int64_t id = load_idx(a.idx, a.idx_is_i64, ib + (int64_t)s * K + j);
            const int64_t rw = lo + id;
            if (id < 0 || rw >= hi) continue;
            row[j] = int(rw);
            if (dist_mode) {
                float acc = 0.f;
#pragma unroll
                for (int d = 0; d < DMAX; ++d) {
                    if (d >= D) continue;
                    const float df = loc[d] - KV[rw * a.kp_sn + d];
                    float sq = df * df;
                    asm volatile("" : "+v"(sq));
                    acc = acc + sq;
                }
                d2[j] = acc;
            }
            if (a.mode == AFF_DEFORM_BWD_IDW) {
                wj[j] = __builtin_amdgcn_rcpf(pow_like_fwd(d2[j], praw, ie) + 1e-10f);
                usum += wj[j];
            } else if (a.mode == AFF_DEFORM_BWD_GIVEN) {
                wj[j] = load_any(a.weights, a.w_dtype, wb + (int64_t)s * K + j);
            } else {
                const float dist = a.mode == AFF_DEFORM_BWD_SAMPLE_SQ ? sqrtf(d2[j] + 1e-6f) : sqrtf(d2[j]) + 1e-6f;
                wj[j] = -pw * dist;  // logit for now
                mx = fmaxf(mx, wj[j]);
            }
        }
        float usum_eps = 0.f;
        if (a.mode == AFF_DEFORM_BWD_IDW) {
            usum_eps = usum + 1e-12f;
            const float inv = __builtin_amdgcn_rcpf(usum_eps);
#pragma unroll
            for (int j = 0; j < KMAX; ++j) wj[j] = row[j] >= 0 ? wj[j] * inv : 0.f;  // wj held u_j until here
        } else if (a.mode != AFF_DEFORM_BWD_GIVEN) {
            float esum = 0.f;
#pragma unroll
            for (int j = 0; j < KMAX; ++j) {
                wj[j] = row[j] >= 0 ? __expf(wj[j] - mx) : 0.f;
                esum += wj[j];
            }
            const float inv = 1.f / (esum + 1e-8f);
#pragma unroll
            for (int j = 0; j < KMAX; ++j) wj[j] *= inv;
        }
        // g_j = dL/dw_j and d_attn
        float dattn = 0.f;
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            gj[j] = 0.f;
            if (j >= K || row[j] < 0) continue;
            if (V) {
                float part = 0.f;
                const T *vr = V + (int64_t)row[j] * a.v_sn;
#pragma unroll
                for (int k = 0; k < NCH; ++k) {
                    const int c0 = 8 * (sub + G * k);
                    if (c0 >= a.C) continue;
                    float vv[8];
                    IO::load8(vr + c0, vv);
#pragma unroll
                    for (int i = 0; i < 8; ++i) part += vv[i] * dof[k][i];
                }
                const float dot = group_sum<G>(part);
                dattn += wj[j] * dot;
                gj[j] = aw * dot;
            } else {
                gj[j] = a.d_w_in[dwb + (int64_t)s * K + j];
            }
        }
        const int64_t rs = r * S + s;
        if (sub == 0) {
            if (a.d_attn) a.d_attn[rs] = dattn;
            if (a.d_weights) {
#pragma unroll
                for (int j = 0; j < KMAX; ++j)
                    if (j < K) a.d_weights[rs * K + j] = gj[j];
            }
        }
        // position terms; each pair's bucket key, d_values coefficient and d_kv_pos term
        float dl[DMAX] = {0.f, 0.f, 0.f, 0.f};
        float gw = 0.f;
#pragma unroll
        for (int j = 0; j < KMAX; ++j) gw += wj[j] * gj[j];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            if (j >= K) continue;
            const int64_t pid = rs * K + j;
            const bool put = w.keyed && sub == 0;
            if (put) {
                w.keys[pid] = row[j] >= 0 ? unsigned(((int64_t)b * a.Nkv + row[j]) * a.H + h) : nkeys;
                w.ids[pid] = int(pid);
                w.coef[pid] = aw * wj[j];
            }
            if (!dist_mode) continue;
            float coef = 0.f;  // d(loc) = coef * diff
            if (row[j] >= 0) {
                if (a.mode == AFF_DEFORM_BWD_IDW) {
                    const float u = wj[j] * usum_eps;  // u_j
                    const float dLdu = (gj[j] - gw) / usum_eps;
                    const float pm1 = ie > 0 ? pow_like_fwd(d2[j], praw - 1.f, ie - 1)
                                             : (d2[j] > 0.f ? powf(d2[j], praw - 1.f) : 0.f);
                    const float dudd2 = -praw * pm1 * u * u;
                    coef = 2.f * dLdu * dudd2;
                    if (d2[j] > 0.f) dpow += dLdu * (-logf(d2[j]) * pow_like_fwd(d2[j], praw, ie) * u * u);
                } else {
                    const float dlg = wj[j] * (gj[j] - gw);
                    const float sq = sqrtf(a.mode == AFF_DEFORM_BWD_SAMPLE_SQ ? d2[j] + 1e-6f : d2[j]);
                    const float dist = a.mode == AFF_DEFORM_BWD_SAMPLE_SQ ? sq : sq + 1e-6f;
                    dpow += dlg * (-dist);
                    const float ddist = -pw * dlg;
                    float den;
                    if (a.mode == AFF_DEFORM_BWD_SHEPARD) den = dist;
                    else if (a.mode == AFF_DEFORM_BWD_SAMPLE) den = fmaxf(dist - 1e-6f, 1e-8f);
                    else den = dist + 1e-8f;
                    coef = ddist / den;
                }
            }
#pragma unroll
            for (int d = 0; d < DMAX; ++d) {
                if (d >= D) continue;
                const float t = row[j] >= 0 ? coef * (loc[d] - KV[(int64_t)row[j] * a.kp_sn + d]) : 0.f;
                dl[d] += t;
                if (put) w.gkv[pid * D + d] = -t;
            }
        }
        if (dist_mode && sub == 0 && a.d_loc) {
#pragma unroll
            for (int d = 0; d < DMAX; ++d)
                if (d < D) a.d_loc[rs * D + d] = dl[d];
        }
    }
    if (sub == 0 && w.dpow_row) w.dpow_row[r] = dpow;
}

// d_values[b, n, h, :] = sum over the bucket's pairs of coef * dout[row of the pair].
template <typename T, int G, int NCH>
__global__ __launch_bounds__(THREADS) void dvalues_kernel(const aff_deform_bwd_args a, const int *ids, const float *coef,
                                                          const int *off) {
    using IO = ElemIO<T>;
    constexpr int RPB = THREADS / G;
    const int sub = threadIdx.x % G;
    const int64_t t = (int64_t)blockIdx.x * RPB + threadIdx.x / G;
    const int64_t T_ = (int64_t)a.B * a.Nkv * a.H;
    if (t >= T_) return;
    const int h = int(t % a.H);
    const int64_t bn = t / a.H;
    const int n = int(bn % a.Nkv), b = int(bn / a.Nkv);
    float acc[NCH][8];
#pragma unroll
    for (int k = 0; k < NCH; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[k][i] = 0.f;
    const int e0 = off[t], e1 = off[t + 1];
    const int SK = a.S * a.K;
    for (int e = e0; e < e1; ++e) {
        const int pid = ids[e];
        const float c = coef[pid];
        const int64_t r = pid / SK;  // (b, q, h) row of the pair
        const int q = int((r / a.H) % a.Q);
        const T *dr = static_cast<const T *>(a.dout) + (int64_t)b * a.do_sb + (int64_t)q * a.do_sn + (int64_t)h * a.do_sh;
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int c0 = 8 * (sub + G * k);
            if (c0 >= a.C) continue;
            float dv[8];
            IO::load8(dr + c0, dv);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[k][i] += c * dv[i];
        }
    }
    T *o = static_cast<T *>(a.d_values) + (((int64_t)b * a.Nkv + n) * a.H + h) * a.C;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c0 = 8 * (sub + G * k);
        if (c0 < a.C) IO::store8(o + c0, acc[k]);
    }
}

// d_kv_pos[b, n, :] = sum over the point's H buckets (in head order) of the pair terms.
__global__ __launch_bounds__(THREADS) void dkv_kernel(const aff_deform_bwd_args a, const int *ids, const float *gkv,
                                                      const int *off) {
    const int64_t p = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    if (p >= (int64_t)a.B * a.Nkv) return;
    float acc[DMAX] = {0.f, 0.f, 0.f, 0.f};
    const int e0 = off[p * a.H], e1 = off[p * a.H + a.H];
    for (int e = e0; e < e1; ++e) {
        const int64_t pid = ids[e];
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < a.D) acc[d] += gkv[pid * a.D + d];
    }
#pragma unroll
    for (int d = 0; d < DMAX; ++d)
        if (d < a.D) a.d_kv_pos[p * a.D + d] = acc[d];
}

// Fixed-order sum of n floats: SUM_CHUNKS partial sums (a block each, LDS tree), then one final block.
__global__ __launch_bounds__(THREADS) void sum_partial_kernel(const float *x, int64_t n, float *part) {
    __shared__ float red[THREADS];
    const int64_t per = (n + gridDim.x - 1) / gridDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * per, i1 = i0 + per < n ? i0 + per : n;
    float s = 0.f;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += THREADS) s += x[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = THREADS / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

__global__ __launch_bounds__(THREADS) void sum_final_kernel(const float *part, int chunks, float *out) {
    __shared__ float red[THREADS];
    float s = 0.f;
    for (int i = threadIdx.x; i < chunks; i += THREADS) s += part[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = THREADS / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = red[0];
}

__global__ __launch_bounds__(THREADS) void zero_kernel(uint8_t *p, int64_t bytes) {
    for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < bytes; i += (int64_t)gridDim.x * THREADS) p[i] = 0;
}

// ------------------------------------------------------------------ host --
inline void fill_zero(void *p, int64_t bytes, hipStream_t s) {
    if (bytes <= 0) return;
    const int64_t blocks = (bytes + THREADS - 1) / THREADS;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(THREADS), 0, s,
                       static_cast<uint8_t *>(p), bytes);
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct Layout {
    size_t keys_in, ids_in, keys_out, ids_out, coef, gkv, off, dpow_row, dpow_part, temp, total, temp_bytes;
    bool keyed;
};

inline int64_t pair_count(const aff_deform_bwd_args &a) { return (int64_t)a.B * a.Q * a.H * a.S * a.K; }

inline Layout layout(const aff_deform_bwd_args &a) {
    Layout L{};
    const int64_t pairs = pair_count(a), rows = (int64_t)a.B * a.Q * a.H;
    const int64_t nkeys = (int64_t)a.B * a.Nkv * a.H;
    L.keyed = (a.d_values && a.values) || (a.d_kv_pos && a.mode != AFF_DEFORM_BWD_GIVEN);
    size_t o = 0;
    auto take = [&](size_t bytes) { const size_t at = o; o = align256(o + bytes); return at; };
    if (L.keyed) {
        L.keys_in = take(pairs * 4);
        L.ids_in = take(pairs * 4);
        L.keys_out = take(pairs * 4);
        L.ids_out = take(pairs * 4);
        L.coef = take(pairs * 4);
        L.gkv = take(pairs * 4 * (a.D > 0 ? a.D : 1));
        L.off = take((nkeys + 1) * 4);
        L.temp_bytes = bucket::sort_temp_bytes(pairs, bucket::key_bits(nkeys));
        L.temp = take(L.temp_bytes);
    }
    L.dpow_row = take(rows * 4);
    L.dpow_part = take(SUM_CHUNKS * 4);
    L.total = o;
    return L;
}

inline int lanes_for(int C) {
    int g = 1;
    while (g < 64 && 8 * g < C) g <<= 1;
    return g;
}

using RowsFn = void (*)(aff_deform_bwd_args, Work);
using DvFn = void (*)(aff_deform_bwd_args, const int *, const float *, const int *);

template <typename T, int G>
RowsFn rows_fn(int nch) {
    if (nch == 0) return rows_kernel<T, G, 0>;
    if (nch == 1) return rows_kernel<T, G, 1>;
    if (nch == 2) return rows_kernel<T, G, 2>;
    return rows_kernel<T, G, NCHMAX>;
}

template <typename T>
RowsFn pick_rows(int G, int nch) {
    switch (G) {
        case 1: return rows_fn<T, 1>(nch);
        case 2: return rows_fn<T, 2>(nch);
        case 4: return rows_fn<T, 4>(nch);
        case 8: return rows_fn<T, 8>(nch);
        case 16: return rows_fn<T, 16>(nch);
        case 32: return rows_fn<T, 32>(nch);
        default: return rows_fn<T, 64>(nch);
    }
}

template <typename T, int G>
DvFn dv_fn(int nch) {
    if (nch <= 1) return dvalues_kernel<T, G, 1>;
    if (nch == 2) return dvalues_kernel<T, G, 2>;
    return dvalues_kernel<T, G, NCHMAX>;
}

template <typename T>
DvFn pick_dv(int G, int nch) {
    switch (G) {
        case 1: return dv_fn<T, 1>(nch);
        case 2: return dv_fn<T, 2>(nch);
        case 4: return dv_fn<T, 4>(nch);
        case 8: return dv_fn<T, 8>(nch);
        case 16: return dv_fn<T, 16>(nch);
        case 32: return dv_fn<T, 32>(nch);
        default: return dv_fn<T, 64>(nch);
    }
}

inline aff_status check_args(const aff_deform_bwd_args &a) {
    AFF_CHECK_ARG(a.mode >= AFF_DEFORM_BWD_SHEPARD && a.mode <= AFF_DEFORM_BWD_GIVEN, "aff_deform_bwd: mode %d", a.mode);
    AFF_CHECK_ARG(a.B >= 0 && a.Q >= 0 && a.H >= 1 && a.S >= 1 && a.K >= 1 && a.Nkv >= 0 && a.P >= 1,
                  "aff_deform_bwd: sizes B=%d Q=%d H=%d S=%d K=%d Nkv=%d P=%d", a.B, a.Q, a.H, a.S, a.K, a.Nkv, a.P);
    if (a.K > KMAX) return fail(AFF_ERR_UNSUPPORTED, "aff_deform_bwd: K=%d above %d", a.K, KMAX);
    const bool dist = a.mode != AFF_DEFORM_BWD_GIVEN;
    AFF_CHECK_ARG(!dist || (a.D >= 1 && a.D <= DMAX), "aff_deform_bwd: D=%d (1..%d)", a.D, DMAX);
    AFF_CHECK_ARG(!dist || (a.loc && a.kv_pos && a.power), "aff_deform_bwd: distance modes need loc, kv_pos, power");
    AFF_CHECK_ARG(dist || a.weights, "aff_deform_bwd: GIVEN mode needs weights");
    AFF_CHECK_ARG(dist || (!a.d_loc && !a.d_kv_pos && !a.d_power), "aff_deform_bwd: GIVEN mode has no position gradients");
    AFF_CHECK_ARG(a.idx, "aff_deform_bwd: NULL idx");
    AFF_CHECK_ARG(a.values || a.d_w_in, "aff_deform_bwd: values or d_w_in is required");
    AFF_CHECK_ARG(!a.values || a.dout, "aff_deform_bwd: values given without dout");
    AFF_CHECK_ARG(!a.d_values || a.values, "aff_deform_bwd: d_values needs values");
    AFF_CHECK_ARG(!a.d_attn || a.values, "aff_deform_bwd: d_attn needs values");
    const int L = (a.S + a.P - 1) / a.P;
    AFF_CHECK_ARG(L <= AFF_DEFORM_MAX_LEVELS && a.level_start[0] == 0, "aff_deform_bwd: levels");
    for (int l = 0; l < L; ++l)
        AFF_CHECK_ARG(a.level_start[l] <= a.level_start[l + 1], "aff_deform_bwd: level_start not non-decreasing");
    AFF_CHECK_ARG(a.level_start[L] <= a.Nkv, "aff_deform_bwd: level_start[%d]=%d beyond Nkv=%d", L, a.level_start[L], a.Nkv);
    if (a.values) {
        AFF_CHECK_ARG(a.dtype == AFF_F32 || a.dtype == AFF_BF16 || a.dtype == AFF_F16, "aff_deform_bwd: dtype");
        AFF_CHECK_ARG(a.C >= 8 && a.C % 8 == 0, "aff_deform_bwd: C=%d must be a positive multiple of 8", a.C);
        if (a.C > 8 * 64 * NCHMAX) return fail(AFF_ERR_UNSUPPORTED, "aff_deform_bwd: C=%d above %d", a.C, 8 * 64 * NCHMAX);
        const int es = a.dtype == AFF_F32 ? 4 : 2;
        const bool al = (reinterpret_cast<uintptr_t>(a.values) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.dout) & 15) == 0 &&
                        (a.v_sb * es) % 16 == 0 && (a.v_sn * es) % 16 == 0 && (a.v_sh * es) % 16 == 0 &&
                        (a.do_sb * es) % 16 == 0 && (a.do_sn * es) % 16 == 0 && (a.do_sh * es) % 16 == 0 &&
                        (!a.d_values || (reinterpret_cast<uintptr_t>(a.d_values) & 15) == 0);
        AFF_CHECK_ARG(al, "aff_deform_bwd: values / dout / d_values rows must be 16-byte aligned");
    }
    AFF_CHECK_ARG(pair_count(a) < (int64_t(1) << 31), "aff_deform_bwd: %lld pairs (limit 2^31)", (long long)pair_count(a));
    AFF_CHECK_ARG((int64_t)a.B * a.Nkv * a.H < (int64_t(1) << 31) - 1, "aff_deform_bwd: too many value rows");
    return AFF_OK;
}

}  // namespace dbwd
}  // namespace aff

using namespace aff;
using namespace aff::dbwd;

extern "C" size_t aff_deform_bwd_workspace_bytes(const aff_deform_bwd_args *args) {
    if (!args) return 0;
    return layout(*args).total;
}

extern "C" aff_status aff_deform_bwd(const aff_deform_bwd_args *args, void *ws, size_t ws_bytes, aff_stream_t stream) {
    AFF_CHECK_ARG(args, "aff_deform_bwd: NULL args");
    const aff_deform_bwd_args &a = *args;
    aff_status st = check_args(a);
    if (st != AFF_OK) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t rows = (int64_t)a.B * a.Q * a.H;
    if (rows == 0) {
        // nothing flows back: zero what was asked for (fill kernels, so that a captured graph replays them)
        if (a.d_kv_pos) fill_zero(a.d_kv_pos, (int64_t)a.B * a.Nkv * a.D * 4, s);
        if (a.d_values) fill_zero(a.d_values, (int64_t)a.B * a.Nkv * a.H * a.C * (a.dtype == AFF_F32 ? 4 : 2), s);
        if (a.d_power) fill_zero(a.d_power, 4, s);
        return check_launch("aff_deform_bwd");
    }
    const Layout L = layout(a);
    if (!ws || ws_bytes < L.total)
        return fail(AFF_ERR_WORKSPACE, "aff_deform_bwd: workspace %zu bytes, need %zu", ws_bytes, L.total);
    char *base = static_cast<char *>(ws);
    Work w{};
    w.keyed = L.keyed;
    if (L.keyed) {
        w.keys = reinterpret_cast<unsigned *>(base + L.keys_in);
        w.ids = reinterpret_cast<int *>(base + L.ids_in);
        w.coef = reinterpret_cast<float *>(base + L.coef);
        w.gkv = reinterpret_cast<float *>(base + L.gkv);
    }
    w.dpow_row = reinterpret_cast<float *>(base + L.dpow_row);

    const int G = a.values ? lanes_for(a.C) : 1;
    const int nch = a.values ? (a.C + 8 * G - 1) / (8 * G) : 0;
    const int rpb = THREADS / G;
    RowsFn rf = a.dtype == AFF_BF16 ? pick_rows<bf16_t>(G, nch)
                : a.dtype == AFF_F16 ? pick_rows<f16_t>(G, nch)
                                     : pick_rows<float>(G, nch);
    hipLaunchKernelGGL(rf, dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(THREADS), 0, s, a, w);
    st = check_launch("aff_deform_bwd rows");
    if (st != AFF_OK) return st;

    if (L.keyed) {
        const int64_t pairs = pair_count(a);
        const int nkeys = int((int64_t)a.B * a.Nkv * a.H);
        unsigned *keys_out = reinterpret_cast<unsigned *>(base + L.keys_out);
        int *ids_out = reinterpret_cast<int *>(base + L.ids_out);
        int *off = reinterpret_cast<int *>(base + L.off);
        st = bucket::sort_and_offsets(w.keys, w.ids, keys_out, ids_out, pairs, nkeys, base + L.temp, L.temp_bytes, off, s);
        if (st != AFF_OK) return st;
        if (a.d_values && a.values && nkeys > 0) {
            DvFn df = a.dtype == AFF_BF16 ? pick_dv<bf16_t>(G, nch)
                      : a.dtype == AFF_F16 ? pick_dv<f16_t>(G, nch)
                                           : pick_dv<float>(G, nch);
            hipLaunchKernelGGL(df, dim3((unsigned)((nkeys + rpb - 1) / rpb)), dim3(THREADS), 0, s, a, ids_out, w.coef, off);
            st = check_launch("aff_deform_bwd d_values");
            if (st != AFF_OK) return st;
        }
        if (a.d_kv_pos && a.mode != AFF_DEFORM_BWD_GIVEN) {
            const int64_t pts = (int64_t)a.B * a.Nkv;
            if (pts > 0) {
                hipLaunchKernelGGL(dkv_kernel, dim3((unsigned)((pts + THREADS - 1) / THREADS)), dim3(THREADS), 0, s, a,
                                   ids_out, w.gkv, off);
                st = check_launch("aff_deform_bwd d_kv_pos");
                if (st != AFF_OK) return st;
            }
        }
    }
    if (a.d_power) {
        float *part = reinterpret_cast<float *>(base + L.dpow_part);
        hipLaunchKernelGGL(sum_partial_kernel, dim3(SUM_CHUNKS), dim3(THREADS), 0, s, w.dpow_row, rows, part);
        hipLaunchKernelGGL(sum_final_kernel, dim3(1), dim3(THREADS), 0, s, part, SUM_CHUNKS, a.d_power);
        st = check_launch("aff_deform_bwd d_power");
    }
    return st;
}
