// LayerNorm for the AFF encoder's glue (the reference's nn.LayerNorm uses and
// LayerNorm2dImages, src/layers/aff.py:96, 108, 296, 494, 514-526, 726):
//
//   y = (x - mean) / sqrt(var + eps) * weight + bias,
//   mean and (biased) var over the normalised dimension, in fp32.
//
// Rows ([rows, C], C % 8 == 0): a group of L = min(64, next_pow2(C / 8)) lanes
// owns one row; lane k holds channels 8 k, 8 k + 8 L, ... in registers (1, 2
// or MAXCH chunks of 8, the fewest that cover C), so mean and variance are
// exact two-pass sums over registers after one read of x.
//
// Maps ([B, C, H, W]): one lane per pixel holds its C channels in registers
// (C <= 64); the loads of a wave are 64 consecutive pixels of one channel.
// The masked patch embedding (aff.py:591-632) is fused in: the map is first
// multiplied by the token keep mask (one value per cell x cell block of
// pixels), the exact-erf GELU may follow the normalisation, and the result is
// written either as [B, C, H, W] or token-major as [B, H * W, C].
#include "common.hpp"

namespace aff {
namespace ln {

constexpr int THREADS = 256;
constexpr int MAXCH = 8;    // chunks of 8 channels per lane: rows of C <= 8 * 64 * MAXCH = 4096
constexpr int MAP_MAXC = 64;

template <typename T>
__device__ __forceinline__ void store1(T *p, float v) {
    if constexpr (sizeof(T) == 4) *reinterpret_cast<float *>(p) = v;
    else if constexpr (__is_same(T, bf16_t)) *reinterpret_cast<uint16_t *>(p) = f32_to_bf16(v);
    else *reinterpret_cast<_Float16 *>(p) = _Float16(v);
}

// Eight consecutive fp32 affine parameters (32-byte aligned: c0 % 8 == 0 and
// the vector itself 16-byte aligned, checked on the host), or `dflt` without one.
__device__ __forceinline__ void load_affine8(const float *p, int c0, float dflt, float (&o)[8]) {
    if (!p) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = dflt;
        return;
    }
    const float4 a = *reinterpret_cast<const float4 *>(p + c0), b = *reinterpret_cast<const float4 *>(p + c0 + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }

// x [rows, C] (row stride xs, unit channel stride), y [rows, C] (row stride ys).
template <typename TI, typename TO, int L, int NCH>
__global__ __launch_bounds__(THREADS) void ln_rows_kernel(const TI *x, int64_t xs, TO *y, int64_t ys,
                                                          const float *w, const float *bias, int64_t rows, int C,
                                                          float eps) {
    const int sub = threadIdx.x % L;
    const int64_t row = (int64_t)blockIdx.x * (THREADS / L) + threadIdx.x / L;
    if (row >= rows) return;  // whole lane groups leave together
    const TI *xr = x + row * xs;
    float v[NCH][8];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c0 = 8 * (sub + L * k);
        if (c0 < C) {
            ElemIO<TI>::load8(xr + c0, v[k]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) s += v[k][i];
    }
    const float mean = group_sum<L>(s) / float(C);
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        if (8 * (sub + L * k) >= C) continue;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float d = v[k][i] - mean;
            q += d * d;
        }
    }
    const float rstd = rsqrtf(group_sum<L>(q) / float(C) + eps);
    TO *yr = y + row * ys;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c0 = 8 * (sub + L * k);
        if (c0 >= C) continue;
        float wv[8], bv[8], o[8];
        load_affine8(w, c0, 1.f, wv);
        load_affine8(bias, c0, 0.f, bv);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (v[k][i] - mean) * rstd * wv[i] + bv[i];
        ElemIO<TO>::store8(yr + c0, o);
    }
}

struct MapArgs {
    const void *x;       // [B, C, H, W]
    void *y;             // [B, C, H, W], or [B, H * W, C] when token_major
    const float *w, *b;  // [C] or NULL
    const float *keep;   // [B, (H / cell) * (W / cell)] token keep mask, or NULL
    int B, C, H, W, cell, token_major, gelu;
    float eps;
};

// One lane per pixel; channels in registers.  Grid: (pixel blocks of one image, B);
// pixel offsets inside one image are 32-bit (host-checked), so the pixel's row,
// column and token need only 32-bit divisions.  MC >= C channels are compiled in:
// every channel load is unconditional (channels past C re-read channel C - 1 and
// are dropped), so a lane's loads are all in flight together.
template <typename TI, typename TO, int MC>
__global__ __launch_bounds__(THREADS) void ln_map_kernel(MapArgs a) {
    const int HW = a.H * a.W;
    const int pix = int(blockIdx.x) * THREADS + int(threadIdx.x);
    if (pix >= HW) return;
    const int64_t b = blockIdx.y;
    const int64_t p = b * HW + pix;
    const int C = a.C;
    const TI *xp = static_cast<const TI *>(a.x) + b * C * HW + pix;
    float kv = 1.f;
    if (a.keep) {
        const int yy = pix / a.W, xx = pix - yy * a.W, tw = a.W / a.cell;
        kv = a.keep[b * (int64_t)(a.H / a.cell) * tw + (yy / a.cell) * tw + xx / a.cell];
    }
    float v[MC];
#pragma unroll
    for (int c = 0; c < MC; ++c) v[c] = ElemIO<TI>::load1(xp + (int64_t)(c < C ? c : C - 1) * HW);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < MC; ++c) {
        v[c] = c < C ? v[c] * kv : 0.f;
        s += v[c];
    }
    const float mean = s / float(C);
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < MC; ++c) {
        const float d = c < C ? v[c] - mean : 0.f;
        q += d * d;
    }
    const float rstd = rsqrtf(q / float(C) + a.eps);
#pragma unroll
    for (int c = 0; c < MC; ++c) {
        const int cc = c < C ? c : 0;
        v[c] = (v[c] - mean) * rstd * (a.w ? a.w[cc] : 1.f) + (a.b ? a.b[cc] : 0.f);
    }
    if (a.gelu) {
#pragma unroll
        for (int c = 0; c < MC; ++c)
            if (c < C) v[c] = gelu_erf(v[c]);
    }
    TO *y = static_cast<TO *>(a.y);
    if (a.token_major) {
        TO *yp = y + p * C;
        if (C % 8 == 0) {
#pragma unroll
            for (int c0 = 0; c0 < MC; c0 += 8) {
                if (c0 >= C) break;
                float o[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = v[c0 + i];
                ElemIO<TO>::store8(yp + c0, o);
            }
        } else {
#pragma unroll
            for (int c = 0; c < MC; ++c)
                if (c < C) store1(yp + c, v[c]);
        }
    } else {
        TO *yp = y + b * C * HW + pix;
#pragma unroll
        for (int c = 0; c < MC; ++c)
            if (c < C) store1(yp + (int64_t)c * HW, v[c]);
    }
}

using RowsFn = void (*)(const void *, int64_t, void *, int64_t, const float *, const float *, int64_t, int, float);
using MapFn = void (*)(MapArgs);

template <typename TI, typename TO, int L>
RowsFn rows_fn(int nch) {
    if (nch == 1) return reinterpret_cast<RowsFn>(ln_rows_kernel<TI, TO, L, 1>);
    if (nch == 2) return reinterpret_cast<RowsFn>(ln_rows_kernel<TI, TO, L, 2>);
    return reinterpret_cast<RowsFn>(ln_rows_kernel<TI, TO, L, MAXCH>);
}

template <typename TI, typename TO>
RowsFn pick_rows_l(int L, int nch) {
    switch (L) {
        case 1: return rows_fn<TI, TO, 1>(nch);
        case 2: return rows_fn<TI, TO, 2>(nch);
        case 4: return rows_fn<TI, TO, 4>(nch);
        case 8: return rows_fn<TI, TO, 8>(nch);
        case 16: return rows_fn<TI, TO, 16>(nch);
        case 32: return rows_fn<TI, TO, 32>(nch);
        default: return rows_fn<TI, TO, 64>(nch);
    }
}

template <typename TI>
RowsFn pick_rows_o(int odt, int L, int nch) {
    if (odt == AFF_F32) return pick_rows_l<TI, float>(L, nch);
    if (odt == AFF_BF16) return pick_rows_l<TI, bf16_t>(L, nch);
    return pick_rows_l<TI, f16_t>(L, nch);
}

template <typename TI, typename TO>
MapFn pick_map_c(int C) {
    if (C <= 16) return reinterpret_cast<MapFn>(ln_map_kernel<TI, TO, 16>);
    if (C <= 32) return reinterpret_cast<MapFn>(ln_map_kernel<TI, TO, 32>);
    return reinterpret_cast<MapFn>(ln_map_kernel<TI, TO, MAP_MAXC>);
}

template <typename TI>
MapFn pick_map_o(int odt, int C) {
    if (odt == AFF_F32) return pick_map_c<TI, float>(C);
    if (odt == AFF_BF16) return pick_map_c<TI, bf16_t>(C);
    return pick_map_c<TI, f16_t>(C);
}

inline bool dtype_ok(int d) { return d == AFF_F32 || d == AFF_BF16 || d == AFF_F16; }

}  // namespace ln
}  // namespace aff

using namespace aff;

extern "C" aff_status aff_layer_norm_fwd(const void *x, int x_dtype, int64_t x_rs, void *y, int y_dtype, int64_t y_rs,
                                         const float *weight, const float *bias, int64_t rows, int C, float eps,
                                         aff_stream_t stream) {
    AFF_CHECK_ARG(rows >= 0 && C >= 1, "aff_layer_norm_fwd: rows=%lld C=%d", (long long)rows, C);
    AFF_CHECK_ARG(ln::dtype_ok(x_dtype) && ln::dtype_ok(y_dtype), "aff_layer_norm_fwd: dtype");
    int L = 1;
    while (L < 64 && 8 * L < C) L <<= 1;
    if (C > 8 * L * ln::MAXCH)
        return fail(AFF_ERR_UNSUPPORTED, "aff_layer_norm_fwd: C=%d above %d", C, 8 * 64 * ln::MAXCH);
    if (rows == 0) return AFF_OK;
    AFF_CHECK_ARG(x && y, "aff_layer_norm_fwd: NULL x/y");
    const int esx = x_dtype == AFF_F32 ? 4 : 2, esy = y_dtype == AFF_F32 ? 4 : 2;
    const bool vec = C % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
                     (x_rs * esx) % 16 == 0 && (y_rs * esy) % 16 == 0;
    AFF_CHECK_ARG(vec, "aff_layer_norm_fwd: C %% 8 == 0 and 16-byte aligned rows are required");
    AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(weight) & 15) == 0 && (reinterpret_cast<uintptr_t>(bias) & 15) == 0,
                  "aff_layer_norm_fwd: weight / bias must be 16-byte aligned");
    const int nch = (C + 8 * L - 1) / (8 * L);  // chunks of 8 channels per lane
    ln::RowsFn fn = x_dtype == AFF_F32    ? ln::pick_rows_o<float>(y_dtype, L, nch)
                    : x_dtype == AFF_BF16 ? ln::pick_rows_o<bf16_t>(y_dtype, L, nch)
                                          : ln::pick_rows_o<f16_t>(y_dtype, L, nch);
    const int rpb = ln::THREADS / L;
    hipLaunchKernelGGL(fn, dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(ln::THREADS), 0, static_cast<hipStream_t>(stream),
                       x, x_rs, y, y_rs, weight, bias, rows, C, eps);
    return check_launch("aff_layer_norm_fwd");
}

extern "C" aff_status aff_layer_norm_map_fwd(const void *x, int x_dtype, void *y, int y_dtype, const float *weight,
                                             const float *bias, const float *keep, int cell, int B, int C, int H,
                                             int W, int token_major, int gelu, float eps, aff_stream_t stream) {
    AFF_CHECK_ARG(B >= 0 && C >= 1 && H >= 0 && W >= 0, "aff_layer_norm_map_fwd: B=%d C=%d H=%d W=%d", B, C, H, W);
    AFF_CHECK_ARG(ln::dtype_ok(x_dtype) && ln::dtype_ok(y_dtype), "aff_layer_norm_map_fwd: dtype");
    if (C > ln::MAP_MAXC)
        return fail(AFF_ERR_UNSUPPORTED, "aff_layer_norm_map_fwd: C=%d above %d", C, ln::MAP_MAXC);
    AFF_CHECK_ARG(!keep || (cell >= 1 && H % cell == 0 && W % cell == 0),
                  "aff_layer_norm_map_fwd: keep mask needs cell >= 1 dividing H=%d and W=%d (cell=%d)", H, W, cell);
    const int64_t pix = (int64_t)B * H * W;
    if (pix == 0) return AFF_OK;
    AFF_CHECK_ARG(x && y, "aff_layer_norm_map_fwd: NULL x/y");
    if (token_major && C % 8 == 0)
        AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(y) & 15) == 0, "aff_layer_norm_map_fwd: y must be 16-byte aligned");
    ln::MapArgs a{x, y, weight, bias, keep, B, C, H, W, keep ? cell : 1, token_major ? 1 : 0, gelu ? 1 : 0, eps};
    ln::MapFn fn = x_dtype == AFF_F32    ? ln::pick_map_o<float>(y_dtype, C)
                   : x_dtype == AFF_BF16 ? ln::pick_map_o<bf16_t>(y_dtype, C)
                                         : ln::pick_map_o<f16_t>(y_dtype, C);
    AFF_CHECK_ARG((int64_t)H * W < ((int64_t)1 << 31) - ln::THREADS && B <= 65535,
                  "aff_layer_norm_map_fwd: H*W=%lld or B=%d too large", (long long)H * W, B);
    hipLaunchKernelGGL(fn, dim3((unsigned)(((int64_t)H * W + ln::THREADS - 1) / ln::THREADS), (unsigned)B),
                       dim3(ln::THREADS), 0, static_cast<hipStream_t>(stream), a);
    return check_launch("aff_layer_norm_map_fwd");
}
