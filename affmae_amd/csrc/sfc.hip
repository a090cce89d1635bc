// Space-filling-curve ordering of tokens for the balanced clustering
// (reference src/utils/geometry.py:170-460).
//
// aff_sfc_curve_keys: one lane per token computes its curve key on an h x w
//   canvas: the alternating scanline index, or the Peano / Hilbert index of
//   calculate_peano_order / calculate_hilbert_order (geometry.py:322-460),
//   with the arithmetic the reference's torch ops perform on the GPU: a
//   position is cut into base-3 (base-2) digits level by level with
//   digit = floor(rem * (1 / cur_h)) and rem = fmod(rem, cur_h) in fp32, and
//   the per-level orders are summed in fp32 as orders[L-1] + sum_i orders[i] *
//   base^2^(L-1-i), in that order.
// aff_sfc_anchor_keys: the anchor ordering (geometry.py:199-268): a token's
//   key is rank(patch) * (max ratio + 1) + ratio with ratio = |p - prev|^2 /
//   (|p - next|^2 + 1e-5), prev / next the centres of the patches before and
//   after its patch on the curve, the maximum taken over the whole batch.
// aff_sfc_argsort: per-row stable ascending argsort of fp32 keys: one radix
//   sort of 64-bit (row, orderable key bits) keys with the token ids as
//   payload.
#include "common.hpp"

#include <hipcub/device/device_radix_sort.hpp>
#include <math.h>

namespace aff {
namespace sfc {

constexpr int THREADS = 256;
constexpr int PART = 256;  // blocks of the anchor ratio maximum

// Peano tables of geometry.py:341-342, indexed [row y][column x].
__device__ __constant__ float PEANO_ORDER[3][3] = {{2, 3, 8}, {1, 4, 7}, {0, 5, 6}};
__device__ __constant__ float PEANO_FLIP[3][3][2] = {{{1, 1}, {1, -1}, {1, 1}},
                                                     {{-1, 1}, {-1, -1}, {-1, 1}},
                                                     {{1, 1}, {1, -1}, {1, 1}}};
// Hilbert tables of geometry.py:418-425.
__device__ __constant__ float HILBERT_ROT[3][2][2] = {{{-1, 1}, {0, 0}}, {{0, -1}, {0, 1}}, {{1, 0}, {-1, 0}}};
__device__ __constant__ float HILBERT_RES[4][4] = {{0, 3, 1, 2}, {2, 3, 1, 0}, {2, 1, 3, 0}, {0, 1, 3, 2}};

// torch.remainder on fp32 with a positive divisor
__device__ __forceinline__ float remainder_pos(float a, float b) {
    float m = fmodf(a, b);
    if (m != 0.f && m < 0.f) m += b;
    return m;
}

// First-level Peano tables of a wide canvas (geometry.py:344-352): column x of
// the 3 x first_w block is column x % 3 of the base order, mirrored vertically
// in odd thirds, plus 9 per third; the flips repeat the base's first two columns.
__device__ __forceinline__ float peano_order_wide(int x, int y) {
    const int third = x / 3;
    return PEANO_ORDER[(third & 1) ? 2 - y : y][x % 3] + 9.f * float(third);
}

__global__ __launch_bounds__(THREADS) void curve_keys_kernel(const aff_sfc_curve_args a) {
    const int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    if (t >= (int64_t)a.B * a.N) return;
    const int b = int(t / a.N), n = int(t % a.N);
    const float px = a.pos[(int64_t)b * a.p_sb + (int64_t)n * a.p_sn];
    const float py = a.pos[(int64_t)b * a.p_sb + (int64_t)n * a.p_sn + 1];
    if (a.curve == AFF_SFC_SCANLINE) {
        // order_mask[y, x] = (y odd ? w - 1 - x : x) + y * w at the flat id trunc(px + py * w)
        const int64_t id = int64_t(__fadd_rn(px, __fmul_rn(py, float(a.w))));
        const int64_t y = id / a.w, x = id - y * a.w;
        a.keys[t] = float(((y & 1) ? (a.w - 1 - x) : x) + y * a.w);
        return;
    }
    const int L = a.levels;
    int dx[AFF_SFC_MAX_LEVELS], dy[AFF_SFC_MAX_LEVELS];
    float rx = px, ry = py;
#pragma unroll
    for (int l = 0; l < AFF_SFC_MAX_LEVELS; ++l) {
        if (l >= L) break;
        // digits of a position outside the canvas are clamped to its border
        const int hi = a.curve == AFF_SFC_PEANO ? 2 : 1;
        const int hix = (l == 0 && a.first_w > 0) ? a.first_w - 1 : hi;
        dx[l] = min(max(int(floorf(__fmul_rn(rx, a.inv_h[l]))), 0), hix);
        dy[l] = min(max(int(floorf(__fmul_rn(ry, a.inv_h[l]))), 0), hi);
        rx = remainder_pos(rx, a.cur_h[l]);
        ry = remainder_pos(ry, a.cur_h[l]);
    }
    const bool wide = a.first_w > 0;
    float ord[AFF_SFC_MAX_LEVELS];
#pragma unroll
    for (int i = 0; i < AFF_SFC_MAX_LEVELS; ++i) {
        ord[i] = 0.f;
        if (i >= L) continue;
        if (a.curve == AFF_SFC_PEANO) {
            float fx = 1.f, fy = 1.f;
#pragma unroll
            for (int j = 0; j < AFF_SFC_MAX_LEVELS; ++j) {
                if (j >= i) break;
                const int lv = i - j - 1;
                const int cx = (lv == 0 && wide) ? (dx[lv] & 1) : dx[lv];
                fx *= PEANO_FLIP[dy[lv]][cx][0];
                fy *= PEANO_FLIP[dy[lv]][cx][1];
            }
            const int qx = fx > 0.f ? dx[i] : 2 - dx[i];
            const int qy = fy > 0.f ? dy[i] : 2 - dy[i];
            ord[i] = (i == 0 && wide) ? peano_order_wide(qx, qy) : PEANO_ORDER[qy][qx];
        } else {
            float rot = 0.f;
#pragma unroll
            for (int j = 0; j < AFF_SFC_MAX_LEVELS; ++j) {
                if (j >= i) break;
                float cr;
                if (j == 0 && wide) cr = HILBERT_ROT[0][dy[0]][dx[0] & 1];
                else cr = HILBERT_ROT[int(remainder_pos(rot, 3.f))][dy[j]][dx[j]];
                rot = cr + rot;
            }
            ord[i] = HILBERT_RES[int(remainder_pos(rot, 4.f))][dx[i] + dy[i] * 2];
        }
    }
    float key = 0.f;
#pragma unroll
    for (int i = 0; i < AFF_SFC_MAX_LEVELS; ++i)
        if (i == L - 1) key = ord[i];
#pragma unroll
    for (int i = 0; i < AFF_SFC_MAX_LEVELS; ++i) {
        if (i >= L - 1) break;
        key = __fadd_rn(key, __fmul_rn(ord[i], a.level_scale[i]));
    }
    a.keys[t] = key;
}

// Pass 1 of the anchor keys: each token's patch rank and distance ratio, and
// per-block maxima of the ratio.
__global__ __launch_bounds__(THREADS) void anchor_ratio_kernel(const aff_sfc_anchor_args a, int *prank, float *ratio,
                                                               float *part) {
    __shared__ float red[THREADS];
    const int64_t total = (int64_t)a.B * a.N;
    const int64_t per = (total + gridDim.x - 1) / gridDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * per, i1 = i0 + per < total ? i0 + per : total;
    float mx = -INFINITY;
    for (int64_t t = i0 + threadIdx.x; t < i1; t += THREADS) {
        const int b = int(t / a.N), n = int(t % a.N);
        const float px = a.pos[(int64_t)b * a.p_sb + (int64_t)n * a.p_sn];
        const float py = a.pos[(int64_t)b * a.p_sb + (int64_t)n * a.p_sn + 1];
        const float cx = floorf(__fdiv_rn(px, a.plw)), cy = floorf(__fdiv_rn(py, a.plh));
        int64_t cell = int64_t(__fadd_rn(cx, __fmul_rn(cy, float(a.npw))));
        cell = cell < 0 ? 0 : (cell >= a.ncell ? a.ncell - 1 : cell);
        const int r = a.cell_rank[cell];
        const float ax = __fsub_rn(px, a.prev_c[2 * r]), ay = __fsub_rn(py, a.prev_c[2 * r + 1]);
        const float bx = __fsub_rn(px, a.next_c[2 * r]), by = __fsub_rn(py, a.next_c[2 * r + 1]);
        const float dp = __fadd_rn(__fmul_rn(ax, ax), __fmul_rn(ay, ay));
        const float dn = __fadd_rn(__fmul_rn(bx, bx), __fmul_rn(by, by));
        const float q = __fdiv_rn(dp, __fadd_rn(dn, 1e-5f));
        prank[t] = r;
        ratio[t] = q;
        mx = fmaxf(mx, q);
    }
    red[threadIdx.x] = mx;
    __syncthreads();
    for (int s = THREADS / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// Pass 2: key = rank * (max + 1) + ratio.
__global__ __launch_bounds__(THREADS) void anchor_key_kernel(const aff_sfc_anchor_args a, const int *prank,
                                                             const float *ratio, const float *part, int nparts) {
    __shared__ float s_mx1;
    if (threadIdx.x == 0) {
        float mx = -INFINITY;
        for (int i = 0; i < nparts; ++i) mx = fmaxf(mx, part[i]);
        s_mx1 = __fadd_rn(mx, 1.f);
    }
    __syncthreads();
    const int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    if (t >= (int64_t)a.B * a.N) return;
    a.keys[t] = __fadd_rn(__fmul_rn(float(prank[t]), s_mx1), ratio[t]);
}

// Unsigned image of a float that sorts like the float; -0 and +0 tie as in a float compare.
__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t u = f == 0.f ? 0u : __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(THREADS) void sort_keys_kernel(const float *keys, int B, int N, uint64_t *k64,
                                                            int64_t *ids) {
    const int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    if (t >= (int64_t)B * N) return;
    k64[t] = (uint64_t(t / N) << 32) | orderable(keys[t]);
    ids[t] = t % N;
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline int bits_for(int64_t v) {
    int b = 1;
    while (b < 31 && ((int64_t)1 << b) <= v) ++b;
    return b;
}

struct SortLayout {
    size_t k_in, k_out, ids, temp, temp_bytes, total;
};

inline SortLayout sort_layout(int B, int N) {
    SortLayout L{};
    const int64_t n = (int64_t)B * N;
    size_t tb = 0;
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, tb, static_cast<const uint64_t *>(nullptr),
                                       static_cast<uint64_t *>(nullptr), static_cast<const int64_t *>(nullptr),
                                       static_cast<int64_t *>(nullptr), (int)n, 0, 32 + bits_for(B), (hipStream_t)0);
    size_t o = 0;
    L.k_in = o; o = align256(o + 8 * n);
    L.k_out = o; o = align256(o + 8 * n);
    L.ids = o; o = align256(o + 8 * n);
    L.temp = o; L.temp_bytes = tb; o = align256(o + tb);
    L.total = o;
    return L;
}

inline size_t anchor_ws(int B, int N) {
    const int64_t n = (int64_t)B * N;
    return align256(4 * n) + align256(4 * n) + align256(4 * PART);
}

}  // namespace sfc
}  // namespace aff

using namespace aff;
using namespace aff::sfc;

extern "C" aff_status aff_sfc_curve_keys(const aff_sfc_curve_args *args, aff_stream_t stream) {
    AFF_CHECK_ARG(args, "aff_sfc_curve_keys: NULL args");
    const aff_sfc_curve_args &a = *args;
    AFF_CHECK_ARG(a.B >= 0 && a.N >= 0, "aff_sfc_curve_keys: B=%d N=%d", a.B, a.N);
    AFF_CHECK_ARG(a.curve >= AFF_SFC_SCANLINE && a.curve <= AFF_SFC_HILBERT, "aff_sfc_curve_keys: curve %d", a.curve);
    if (a.curve == AFF_SFC_SCANLINE) {
        AFF_CHECK_ARG(a.w >= 1, "aff_sfc_curve_keys: w=%d", a.w);
    } else {
        AFF_CHECK_ARG(a.levels >= 1 && a.levels <= AFF_SFC_MAX_LEVELS, "aff_sfc_curve_keys: levels=%d (1..%d)",
                      a.levels, AFF_SFC_MAX_LEVELS);
        if (a.curve == AFF_SFC_HILBERT && a.first_w > 0)
            return fail(AFF_ERR_UNSUPPORTED,
                        "aff_sfc_curve_keys: the Hilbert order is defined for square canvases only (first_w=%d)",
                        a.first_w);
    }
    const int64_t n = (int64_t)a.B * a.N;
    if (n == 0) return AFF_OK;
    AFF_CHECK_ARG(a.pos && a.keys, "aff_sfc_curve_keys: NULL pos/keys");
    hipLaunchKernelGGL(curve_keys_kernel, dim3((unsigned)((n + THREADS - 1) / THREADS)), dim3(THREADS), 0,
                       static_cast<hipStream_t>(stream), a);
    return check_launch("aff_sfc_curve_keys");
}

extern "C" size_t aff_sfc_anchor_workspace_bytes(int B, int N) { return anchor_ws(B, N); }

extern "C" aff_status aff_sfc_anchor_keys(const aff_sfc_anchor_args *args, void *ws, size_t ws_bytes,
                                          aff_stream_t stream) {
    AFF_CHECK_ARG(args, "aff_sfc_anchor_keys: NULL args");
    const aff_sfc_anchor_args &a = *args;
    AFF_CHECK_ARG(a.B >= 0 && a.N >= 0 && a.npw >= 1 && a.ncell >= 1, "aff_sfc_anchor_keys: sizes");
    const int64_t n = (int64_t)a.B * a.N;
    if (n == 0) return AFF_OK;
    AFF_CHECK_ARG(a.pos && a.keys && a.cell_rank && a.prev_c && a.next_c, "aff_sfc_anchor_keys: NULL pointer");
    const size_t need = anchor_ws(a.B, a.N);
    if (!ws || ws_bytes < need)
        return fail(AFF_ERR_WORKSPACE, "aff_sfc_anchor_keys: workspace %zu bytes, need %zu", ws_bytes, need);
    char *base = static_cast<char *>(ws);
    int *prank = reinterpret_cast<int *>(base);
    float *ratio = reinterpret_cast<float *>(base + align256(4 * n));
    float *part = reinterpret_cast<float *>(base + 2 * align256(4 * n));
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(anchor_ratio_kernel, dim3(PART), dim3(THREADS), 0, s, a, prank, ratio, part);
    hipLaunchKernelGGL(anchor_key_kernel, dim3((unsigned)((n + THREADS - 1) / THREADS)), dim3(THREADS), 0, s, a, prank,
                       ratio, part, PART);
    return check_launch("aff_sfc_anchor_keys");
}

extern "C" size_t aff_sfc_argsort_workspace_bytes(int B, int N) {
    if (B <= 0 || N <= 0) return 0;
    return sort_layout(B, N).total;
}

extern "C" aff_status aff_sfc_argsort(const float *keys, int B, int N, int64_t *ranking, void *ws, size_t ws_bytes,
                                      aff_stream_t stream) {
    AFF_CHECK_ARG(B >= 0 && N >= 0, "aff_sfc_argsort: B=%d N=%d", B, N);
    const int64_t n = (int64_t)B * N;
    if (n == 0) return AFF_OK;
    AFF_CHECK_ARG(keys && ranking, "aff_sfc_argsort: NULL keys/ranking");
    AFF_CHECK_ARG(n < (int64_t(1) << 31), "aff_sfc_argsort: %lld keys (limit 2^31)", (long long)n);
    const SortLayout L = sort_layout(B, N);
    if (!ws || ws_bytes < L.total)
        return fail(AFF_ERR_WORKSPACE, "aff_sfc_argsort: workspace %zu bytes, need %zu", ws_bytes, L.total);
    char *base = static_cast<char *>(ws);
    uint64_t *k_in = reinterpret_cast<uint64_t *>(base + L.k_in);
    uint64_t *k_out = reinterpret_cast<uint64_t *>(base + L.k_out);
    int64_t *ids = reinterpret_cast<int64_t *>(base + L.ids);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(sort_keys_kernel, dim3((unsigned)((n + THREADS - 1) / THREADS)), dim3(THREADS), 0, s, keys, B,
                       N, k_in, ids);
    aff_status st = check_launch("aff_sfc_argsort (keys)");
    if (st != AFF_OK) return st;
    size_t tb = L.temp_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(base + L.temp, tb, k_in, k_out, ids, ranking, (int)n, 0, 32 + bits_for(B),
                                           s) != hipSuccess)
        return fail(AFF_ERR_LAUNCH, "aff_sfc_argsort: radix sort of %lld keys failed", (long long)n);
    return check_launch("aff_sfc_argsort");
}
