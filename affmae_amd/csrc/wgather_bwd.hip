// Weighted neighbour features / weighted gather, backward, for gfx950.
//
// Forward (weighted_features.py:30-111, weighted_gather.py:21-102):
//   out[b, i, ic, c] = sum_m w[b, i, m, ic] * feat[b, idx[b, i, m], c]
// Backward (the gradients weighted_features.py:164-398 and
// weighted_gather.py:127-326 compute, with floating-point atomics for dfeat):
//   dw[b, i, m, ic] = sum_c dout[b, i, ic, c] * feat[b, idx[b, i, m], c]
//   dfeat[b, r, c]  = sum over (i, m) with idx[b, i, m] = r of sum_ic w[b, i, m, ic] dout[b, i, ic, c]
// Indices outside [0, Nsrc) contribute nothing (and get dw = 0).
//
// dw_kernel: one wave per output row (b, i), lanes over channels; for each
// neighbour the IC dot products are summed across the wave.
// dfeat: the (b, i, m) entries are bucketed by source row with the stable
// sort of bucket.hpp, and dfeat_kernel (one wave per source row, lanes over
// channels) walks its bucket in (b, i, m) order, so dfeat is a fixed-order
// sum with no atomics.
#include "bucket.hpp"
#include "common.hpp"

#include <type_traits>

namespace aff {
namespace wgb {

constexpr int THREADS = 256;
constexpr int WAVES = THREADS / 64;
constexpr int MAX_IC = 8;

struct Args {
    const void *dout; int64_t do_sb, do_sn, do_sic;
    const void *w; int w_dtype; int64_t w_sb, w_sn, w_sm, w_sic;
    const void *feat; int64_t f_sb, f_sn;
    const void *idx; int idx_is_i64; int64_t i_sb, i_sn;
    int B, Nout, Nsrc, M, C, IC;
};

__device__ __forceinline__ int64_t load_idx(const Args &a, int b, int i, int m) {
    const int64_t e = (int64_t)b * a.i_sb + (int64_t)i * a.i_sn + m;
    return a.idx_is_i64 ? static_cast<const int64_t *>(a.idx)[e] : int64_t(static_cast<const int32_t *>(a.idx)[e]);
}

template <typename T>
__device__ __forceinline__ float ld(const void *p, int64_t e) {
    return ElemIO<T>::load1(static_cast<const T *>(p) + e);
}

template <typename T>
__device__ __forceinline__ void st(void *p, int64_t e, float v) {
    if constexpr (sizeof(T) == 4) static_cast<float *>(p)[e] = v;
    else if constexpr (std::is_same<T, bf16_t>::value) static_cast<uint16_t *>(p)[e] = f32_to_bf16(v);
    else static_cast<_Float16 *>(p)[e] = _Float16(v);
}

// dw[b, i, m, ic] (contiguous [B, Nout, M, IC], dtype DW).  IC <= MAX_IC.
template <typename T, typename DW>
__global__ __launch_bounds__(THREADS) void dw_kernel(const Args a, void *dw) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * WAVES + (threadIdx.x >> 6);
    if (row >= (int64_t)a.B * a.Nout) return;  // whole waves leave together
    const int b = int(row / a.Nout), i = int(row % a.Nout);
    const int C = a.C, IC = a.IC;
    const int64_t dbase = (int64_t)b * a.do_sb + (int64_t)i * a.do_sn;
    for (int m = 0; m < a.M; ++m) {
        const int64_t r = load_idx(a, b, i, m);
        const bool ok = r >= 0 && r < a.Nsrc;
        float part[MAX_IC];
#pragma unroll
        for (int ic = 0; ic < MAX_IC; ++ic) part[ic] = 0.f;
        if (ok) {
            const int64_t fbase = (int64_t)b * a.f_sb + r * a.f_sn;
            for (int c = lane; c < C; c += 64) {
                const float f = ld<T>(a.feat, fbase + c);
#pragma unroll
                for (int ic = 0; ic < MAX_IC; ++ic)
                    if (ic < IC) part[ic] += f * ld<T>(a.dout, dbase + (int64_t)ic * a.do_sic + c);
            }
        }
#pragma unroll
        for (int ic = 0; ic < MAX_IC; ++ic)
            if (ic < IC) {
                const float s = group_sum<64>(part[ic]);
                if (lane == 0) st<DW>(dw, (row * a.M + m) * IC + ic, ok ? s : 0.f);
            }
    }
}

// Bucket keys: source row b * Nsrc + idx (sentinel B * Nsrc outside the range),
// payload (b * Nout + i) * M + m.
__global__ __launch_bounds__(THREADS) void keys_kernel(const Args a, unsigned *keys, int *vals) {
    const int64_t e = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.Nout * a.M;
    if (e >= total) return;
    const int m = int(e % a.M);
    const int64_t bi = e / a.M;
    const int b = int(bi / a.Nout), i = int(bi % a.Nout);
    const int64_t r = load_idx(a, b, i, m);
    const bool ok = r >= 0 && r < a.Nsrc;
    keys[e] = ok ? unsigned((int64_t)b * a.Nsrc + r) : unsigned((int64_t)a.B * a.Nsrc);
    vals[e] = int(e);
}

// dfeat[b, r, :] (contiguous [B, Nsrc, C], dtype T): one wave per source row.
template <typename T>
__global__ __launch_bounds__(THREADS) void dfeat_kernel(const Args a, const int *vals, const int *off, void *dfeat) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * WAVES + (threadIdx.x >> 6);
    if (row >= (int64_t)a.B * a.Nsrc) return;
    const int C = a.C, IC = a.IC;
    const int lo = off[row], hi = off[row + 1];
    for (int c0 = 0; c0 < C; c0 += 64) {
        const int c = c0 + lane;
        float acc = 0.f;
        for (int e = lo; e < hi; ++e) {
            const int64_t v = vals[e];                       // (b * Nout + i) * M + m
            const int m = int(v % a.M);
            const int64_t bi = v / a.M;
            const int b = int(bi / a.Nout), i = int(bi % a.Nout);
            const int64_t wbase = (int64_t)b * a.w_sb + (int64_t)i * a.w_sn + (int64_t)m * a.w_sm;
            const int64_t dbase = (int64_t)b * a.do_sb + (int64_t)i * a.do_sn;
            if (c < C)
                for (int ic = 0; ic < IC; ++ic)
                    acc += load_any(a.w, a.w_dtype, wbase + (int64_t)ic * a.w_sic) *
                           ld<T>(a.dout, dbase + (int64_t)ic * a.do_sic + c);
        }
        if (c < C) st<T>(dfeat, row * C + c, acc);
    }
}

struct Layout {
    size_t keys_in, vals_in, keys_out, vals_out, off, temp, temp_bytes, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline Layout layout(int B, int Nout, int Nsrc, int M) {
    const int64_t pairs = (int64_t)B * Nout * M;
    Layout L{};
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = align256(o + bytes);
        return at;
    };
    L.keys_in = take(sizeof(unsigned) * pairs);
    L.vals_in = take(sizeof(int) * pairs);
    L.keys_out = take(sizeof(unsigned) * pairs);
    L.vals_out = take(sizeof(int) * pairs);
    L.off = take(sizeof(int) * ((int64_t)B * Nsrc + 1));
    L.temp_bytes = bucket::sort_temp_bytes(pairs, bucket::key_bits((int64_t)B * Nsrc));
    L.temp = take(L.temp_bytes);
    L.total = o;
    return L;
}

template <typename T>
using DwFn = void (*)(const Args, void *);

template <typename T>
DwFn<T> pick_dw(int dw_dtype) {
    if (dw_dtype == AFF_F32) return dw_kernel<T, float>;
    if (dw_dtype == AFF_BF16) return dw_kernel<T, bf16_t>;
    return dw_kernel<T, f16_t>;
}

inline unsigned blocks(int64_t items, int per) { return (unsigned)((items + per - 1) / per); }

}  // namespace wgb
}  // namespace aff

using namespace aff;

extern "C" size_t aff_weighted_features_bwd_workspace_bytes(int B, int Nout, int Nsrc, int M) {
    if (B <= 0 || Nout <= 0 || Nsrc <= 0 || M <= 0) return 0;
    return wgb::layout(B, Nout, Nsrc, M).total;
}

extern "C" aff_status aff_weighted_features_bwd(const void *dout, int64_t do_sb, int64_t do_sn, int64_t do_sic,
                                                const void *weights, int w_dtype, int64_t w_sb, int64_t w_sn,
                                                int64_t w_sm, int64_t w_sic, const void *feat, int f_dtype,
                                                int64_t f_sb, int64_t f_sn, const void *nbhd_idx, int idx_is_i64,
                                                int64_t i_sb, int64_t i_sn, int B, int Nout, int Nsrc, int M, int C,
                                                int IC, void *d_weights, int dw_dtype, void *d_feat, void *ws,
                                                size_t ws_bytes, aff_stream_t stream) {
    AFF_CHECK_ARG(B >= 0 && Nout >= 0 && Nsrc >= 0 && M >= 0 && C >= 0, "aff_weighted_features_bwd: negative size");
    AFF_CHECK_ARG(IC >= 1 && IC <= wgb::MAX_IC, "aff_weighted_features_bwd: IC=%d outside [1, %d]", IC, wgb::MAX_IC);
    auto okd = [](int d) { return d == AFF_F32 || d == AFF_BF16 || d == AFF_F16; };
    AFF_CHECK_ARG(okd(w_dtype) && okd(f_dtype) && okd(dw_dtype), "aff_weighted_features_bwd: dtype");
    if ((int64_t)B * Nout * C == 0 && (int64_t)B * Nsrc * C == 0) return AFF_OK;
    AFF_CHECK_ARG(dout && weights && feat && (M == 0 || nbhd_idx), "aff_weighted_features_bwd: NULL input");
    AFF_CHECK_ARG((int64_t)B * Nout * M < ((int64_t)1 << 31) && (int64_t)B * Nsrc < ((int64_t)1 << 31),
                  "aff_weighted_features_bwd: problem too large");
    const wgb::Args a{dout, do_sb, do_sn, do_sic, weights, w_dtype, w_sb, w_sn, w_sm, w_sic, feat, f_sb, f_sn,
                      nbhd_idx, idx_is_i64, i_sb, i_sn, B, Nout, Nsrc, M, C, IC};
    hipStream_t hs = static_cast<hipStream_t>(stream);
    aff_status s = AFF_OK;
    if (d_weights && (int64_t)B * Nout * M > 0) {
        if (f_dtype == AFF_F32) hipLaunchKernelGGL(wgb::pick_dw<float>(dw_dtype), dim3(wgb::blocks((int64_t)B * Nout, wgb::WAVES)), dim3(wgb::THREADS), 0, hs, a, d_weights);
        else if (f_dtype == AFF_BF16) hipLaunchKernelGGL(wgb::pick_dw<bf16_t>(dw_dtype), dim3(wgb::blocks((int64_t)B * Nout, wgb::WAVES)), dim3(wgb::THREADS), 0, hs, a, d_weights);
        else hipLaunchKernelGGL(wgb::pick_dw<f16_t>(dw_dtype), dim3(wgb::blocks((int64_t)B * Nout, wgb::WAVES)), dim3(wgb::THREADS), 0, hs, a, d_weights);
        if ((s = check_launch("aff_weighted_features_bwd (dw)")) != AFF_OK) return s;
    }
    if (d_feat && (int64_t)B * Nsrc > 0) {
        const wgb::Layout L = wgb::layout(B, Nout, Nsrc, M > 0 ? M : 1);
        AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(ws) & 255) == 0, "aff_weighted_features_bwd: workspace alignment");
        if (ws == nullptr || ws_bytes < L.total)
            return fail(AFF_ERR_WORKSPACE, "aff_weighted_features_bwd: workspace of %zu bytes needed, got %zu", L.total,
                        ws ? ws_bytes : (size_t)0);
        char *w8 = static_cast<char *>(ws);
        unsigned *keys_in = reinterpret_cast<unsigned *>(w8 + L.keys_in), *keys_out = reinterpret_cast<unsigned *>(w8 + L.keys_out);
        int *vals_in = reinterpret_cast<int *>(w8 + L.vals_in), *vals_out = reinterpret_cast<int *>(w8 + L.vals_out);
        int *off = reinterpret_cast<int *>(w8 + L.off);
        const int64_t pairs = (int64_t)B * Nout * M;
        if (pairs > 0) {
            hipLaunchKernelGGL(wgb::keys_kernel, dim3(wgb::blocks(pairs, wgb::THREADS)), dim3(wgb::THREADS), 0, hs, a,
                               keys_in, vals_in);
            if ((s = check_launch("aff_weighted_features_bwd (keys)")) != AFF_OK) return s;
        }
        if ((s = bucket::sort_and_offsets(keys_in, vals_in, keys_out, vals_out, pairs, B * Nsrc, w8 + L.temp,
                                          L.temp_bytes, off, hs)) != AFF_OK)
            return s;
        const dim3 grid(wgb::blocks((int64_t)B * Nsrc, wgb::WAVES));
        if (f_dtype == AFF_F32) hipLaunchKernelGGL(wgb::dfeat_kernel<float>, grid, dim3(wgb::THREADS), 0, hs, a, vals_out, off, d_feat);
        else if (f_dtype == AFF_BF16) hipLaunchKernelGGL(wgb::dfeat_kernel<bf16_t>, grid, dim3(wgb::THREADS), 0, hs, a, vals_out, off, d_feat);
        else hipLaunchKernelGGL(wgb::dfeat_kernel<f16_t>, grid, dim3(wgb::THREADS), 0, hs, a, vals_out, off, d_feat);
        if ((s = check_launch("aff_weighted_features_bwd (dfeat)")) != AFF_OK) return s;
    }
    return AFF_OK;
}
