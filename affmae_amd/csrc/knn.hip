// Exact 2-D K-nearest-neighbour search for gfx950.
//
// Semantics follow the streaming top-K kernels of the reference
// (src/layers/kernels/knn.py:258-337, 422-471): squared Euclidean distance in
// fp32, results in ascending distance, equal distances resolved by the lower
// reference index.  Here the order is made explicit by sorting 64-bit keys
// (float bits of d2 << 32 | index), so it does not depend on visit order.
//
// Instead of streaming every reference point per query (O(M*N)), each image's
// reference points are counting-sorted into a uniform cell grid (one
// workgroup per image, histogram in LDS), and each query visits only the
// cells that can hold points within a radius U.  U is adjusted until the
// number of points with d2 <= U lies in [k, CAP]; those candidates are kept
// in a per-lane LDS list, sorted in registers with a bitonic network and the
// first k written.  A query that cannot reach that window (ties at one
// distance, k > CAP) falls back to k exact "next smallest key" passes.
#include "common.hpp"

#include <math.h>

namespace aff {
namespace knn {

struct GridParams {
    float x0, y0, h, inv_h;
    int gx, gy, ncell, pad;
};

constexpr int BUILD_THREADS = 1024;
constexpr int MAX_CELLS = 16384;  // LDS histogram of the build kernel: 64 KB
constexpr int PTS_PER_CELL = 2;
constexpr int QUERY_THREADS = 64;
constexpr int MAX_REFINE = 64;

inline int target_cells(int N) {
    int c = N / PTS_PER_CELL;
    if (c < 1) c = 1;
    if (c > MAX_CELLS) c = MAX_CELLS;
    return c;
}

struct WsLayout {
    size_t params, cells, pts, total;
    int cmax;
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline WsLayout ws_layout(int B, int N) {
    WsLayout w;
    w.cmax = target_cells(N);
    size_t off = 0;
    w.params = off;
    off = align256(off + sizeof(GridParams) * (size_t)B);
    w.cells = off;
    off = align256(off + sizeof(int) * (size_t)B * (size_t)(w.cmax + 1));
    w.pts = off;
    off = align256(off + sizeof(float4) * (size_t)B * (size_t)N);
    w.total = off;
    return w;
}

// Cell coordinate of v along one axis.  Monotone non-decreasing in v, which
// is what makes "all points with coordinate in [a, b] lie in cells
// [cell(a), cell(b)]" hold exactly under fp32 rounding.
__device__ __forceinline__ int cell_coord(float v, float origin, float inv_h, int g) {
#pragma clang fp contract(off)
    float f = floorf(__fmul_rn(__fsub_rn(v, origin), inv_h));
    f = fminf(fmaxf(f, 0.f), float(g - 1));
    return int(f);
}

// d2 = fl(fl(dx*dx) + fl(dy*dy)): no fused multiply-add, so the value (and
// therefore the tie order) is the one a plain fp32 CPU evaluation gives.
__device__ __forceinline__ float dist2(float ax, float ay, float bx, float by) {
#pragma clang fp contract(off)
    float dx = __fsub_rn(ax, bx);
    float dy = __fsub_rn(ay, by);
    return __fadd_rn(__fmul_rn(dx, dx), __fmul_rn(dy, dy));
}

__device__ __forceinline__ uint64_t make_key(float d2, int idx) {
    return (uint64_t(__float_as_uint(d2)) << 32) | uint32_t(idx);
}

// ------------------------------------------------------------- build ----
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__global__ __launch_bounds__(BUILD_THREADS) void grid_build_kernel(
    const float *__restrict__ ref, int64_t r_sb, int64_t r_sn, int N, int cmax,
    GridParams *__restrict__ gp_out, int *__restrict__ cells_out, float4 *__restrict__ pts_out) {
    __shared__ int s_cnt[MAX_CELLS];
    __shared__ float s_red[4][BUILD_THREADS / 64];
    __shared__ int s_wave[BUILD_THREADS / 64];
    __shared__ GridParams s_gp;

    const int b = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    constexpr int NW = BUILD_THREADS / 64;
    const float *R = ref + (int64_t)b * r_sb;

    // 1. bounding box
    float xmn = INFINITY, xmx = -INFINITY, ymn = INFINITY, ymx = -INFINITY;
    for (int i = tid; i < N; i += BUILD_THREADS) {
        float x = R[(int64_t)i * r_sn], y = R[(int64_t)i * r_sn + 1];
        xmn = fminf(xmn, x); xmx = fmaxf(xmx, x);
        ymn = fminf(ymn, y); ymx = fmaxf(ymx, y);
    }
    xmn = wave_min(xmn); xmx = wave_max(xmx); ymn = wave_min(ymn); ymx = wave_max(ymx);
    if (lane == 0) {
        s_red[0][wid] = xmn; s_red[1][wid] = xmx; s_red[2][wid] = ymn; s_red[3][wid] = ymx;
    }
    __syncthreads();

    // 2. grid parameters (one thread)
    if (tid == 0) {
        for (int w = 1; w < NW; ++w) {
            xmn = fminf(xmn, s_red[0][w]); xmx = fmaxf(xmx, s_red[1][w]);
            ymn = fminf(ymn, s_red[2][w]); ymx = fmaxf(ymx, s_red[3][w]);
        }
        GridParams p;
        p.x0 = xmn; p.y0 = ymn; p.pad = 0;
        float w = xmx - xmn, hh = ymx - ymn;
        float ext = fmaxf(w, hh);
        int gx = 1, gy = 1;
        float h = 1.f;
        if (ext > 0.f && ext < INFINITY) {
            float T = float(cmax);
            float wa = fmaxf(w, ext / T), ha = fmaxf(hh, ext / T);
            h = sqrtf(wa * ha / T);
            for (;;) {
                gx = (int)fminf(w / h + 1.f, T);
                gy = (int)fminf(hh / h + 1.f, T);
                if ((int64_t)gx * gy <= cmax) break;
                h *= 1.0625f;
            }
        } else {
            if (!(xmn > -INFINITY && xmn < INFINITY)) p.x0 = 0.f;
            if (!(ymn > -INFINITY && ymn < INFINITY)) p.y0 = 0.f;
        }
        p.h = h; p.inv_h = 1.f / h; p.gx = gx; p.gy = gy; p.ncell = gx * gy;
        s_gp = p;
        gp_out[b] = p;
    }
    __syncthreads();
    const GridParams p = s_gp;
    const int ncell = p.ncell;

    // 3. histogram
    for (int c = tid; c < ncell; c += BUILD_THREADS) s_cnt[c] = 0;
    __syncthreads();
    for (int i = tid; i < N; i += BUILD_THREADS) {
        float x = R[(int64_t)i * r_sn], y = R[(int64_t)i * r_sn + 1];
        int c = cell_coord(y, p.y0, p.inv_h, p.gy) * p.gx + cell_coord(x, p.x0, p.inv_h, p.gx);
        atomicAdd(&s_cnt[c], 1);
    }
    __syncthreads();

    // 4. exclusive scan: each thread owns a contiguous chunk of cells
    const int chunk = (ncell + BUILD_THREADS - 1) / BUILD_THREADS;
    const int c0 = min(tid * chunk, ncell), c1 = min(c0 + chunk, ncell);
    int local = 0;
    for (int c = c0; c < c1; ++c) local += s_cnt[c];
    int incl = local;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) s_wave[wid] = incl;
    __syncthreads();
    if (wid == 0) {
        int v = lane < NW ? s_wave[lane] : 0;
#pragma unroll
        for (int o = 1; o < NW; o <<= 1) {
            int y = __shfl_up(v, o, 64);
            if (lane >= o) v += y;
        }
        if (lane < NW) s_wave[lane] = v;
    }
    __syncthreads();
    int run = (wid > 0 ? s_wave[wid - 1] : 0) + incl - local;
    int *cells = cells_out + (size_t)b * (cmax + 1);
    for (int c = c0; c < c1; ++c) {
        int n = s_cnt[c];
        cells[c] = run;
        s_cnt[c] = run;  // becomes the scatter cursor
        run += n;
    }
    if (tid == 0) cells[ncell] = N;
    __syncthreads();

    // 5. scatter points into cell order
    float4 *pts = pts_out + (size_t)b * N;
    for (int i = tid; i < N; i += BUILD_THREADS) {
        float x = R[(int64_t)i * r_sn], y = R[(int64_t)i * r_sn + 1];
        int c = cell_coord(y, p.y0, p.inv_h, p.gy) * p.gx + cell_coord(x, p.x0, p.inv_h, p.gx);
        int slot = atomicAdd(&s_cnt[c], 1);
        pts[slot] = make_float4(x, y, __int_as_float(i), 0.f);
    }
}

// ------------------------------------------------------------- query ----
// Calls f(d2, index) for every reference point whose computed d2 can be
// <= U (a superset: whole cells intersecting a slightly enlarged disk).
template <typename F>
__device__ __forceinline__ void visit_disk(const GridParams &p, const int *__restrict__ cs,
                                           const float4 *__restrict__ P, float qx, float qy,
                                           float U, float slack, F &&f) {
    const float r = sqrtf(U) * 1.00002f + slack;
    const int cy0 = cell_coord(qy - r, p.y0, p.inv_h, p.gy);
    const int cy1 = cell_coord(qy + r, p.y0, p.inv_h, p.gy);
    for (int cy = cy0; cy <= cy1; ++cy) {
        const float rlo = p.y0 + float(cy) * p.h, rhi = rlo + p.h;
        const float dy = fmaxf(0.f, fmaxf(rlo - qy, qy - rhi) - slack);
        const float w2 = r * r - dy * dy;
        if (!(w2 >= 0.f)) continue;
        const float w = sqrtf(w2) + slack;
        const int cx0 = cell_coord(qx - w, p.x0, p.inv_h, p.gx);
        const int cx1 = cell_coord(qx + w, p.x0, p.inv_h, p.gx);
        const int beg = cs[cy * p.gx + cx0], end = cs[cy * p.gx + cx1 + 1];
        for (int t = beg; t < end; ++t) {
            const float4 pt = P[t];
            f(dist2(pt.x, pt.y, qx, qy), __float_as_int(pt.z));
        }
    }
}

template <int N>
__device__ __forceinline__ void bitonic_sort(uint64_t (&a)[N]) {
#pragma unroll
    for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    const uint64_t x = a[i], y = a[l];
                    const bool up = (i & k) == 0;
                    const bool sw = up ? (x > y) : (x < y);
                    a[i] = sw ? y : x;
                    a[l] = sw ? x : y;
                }
            }
        }
    }
}

__device__ __forceinline__ void store_result(void *out_idx, int idx_i64, float *out_d2, int64_t o,
                                             uint64_t key) {
    const int idx = int(uint32_t(key));
    if (idx_i64)
        static_cast<int64_t *>(out_idx)[o] = idx;
    else
        static_cast<int32_t *>(out_idx)[o] = idx;
    if (out_d2) out_d2[o] = __uint_as_float(uint32_t(key >> 32));
}

template <int CAP>
__global__ __launch_bounds__(QUERY_THREADS) void knn_query_kernel(
    const float *__restrict__ query, int64_t q_sb, int64_t q_sm,
    const GridParams *__restrict__ gp, const int *__restrict__ cells, const float4 *__restrict__ pts,
    int M, int N, int k, int cmax, void *__restrict__ out_idx, int idx_i64, float *__restrict__ out_d2) {
    __shared__ uint64_t s_list[CAP * QUERY_THREADS];
    const int lane = threadIdx.x;
    const int b = blockIdx.y;
    const int qi = blockIdx.x * QUERY_THREADS + lane;
    if (qi >= M) return;

    const GridParams p = gp[b];
    const int *cs = cells + (size_t)b * (cmax + 1);
    const float4 *P = pts + (size_t)b * N;
    const float *Q = query + (int64_t)b * q_sb + (int64_t)qi * q_sm;
    const float qx = Q[0], qy = Q[1];
    const int64_t obase = ((int64_t)b * M + qi) * k;

    // Slack absorbs fp32 rounding in cell bounds and distances.
    const float gw = float(p.gx) * p.h, gh = float(p.gy) * p.h;
    const float slack = 1e-5f * (fabsf(p.x0) + fabsf(p.y0) + gw + gh + fabsf(qx) + fabsf(qy)) + 1e-30f;

    // Initial radius from the local density of a 5x5 cell window.
    const int cx = cell_coord(qx, p.x0, p.inv_h, p.gx), cy = cell_coord(qy, p.y0, p.inv_h, p.gy);
    const int ax0 = max(cx - 2, 0), ax1 = min(cx + 2, p.gx - 1);
    const int ay0 = max(cy - 2, 0), ay1 = min(cy + 2, p.gy - 1);
    int cntw = 0;
    for (int y = ay0; y <= ay1; ++y) cntw += cs[y * p.gx + ax1 + 1] - cs[y * p.gx + ax0];
    const float h2 = p.h * p.h;
    const float rho = cntw > 0 ? float(cntw) / (float((ax1 - ax0 + 1) * (ay1 - ay0 + 1)) * h2)
                               : float(N) / (float(p.ncell) * h2);
    const float target = 0.5f * float(k + CAP);
    const float ex = fmaxf(0.f, fmaxf(p.x0 - qx, qx - (p.x0 + gw)));
    const float ey = fmaxf(0.f, fmaxf(p.y0 - qy, qy - (p.y0 + gh)));
    float rad = sqrtf(target / (3.14159265f * rho)) + sqrtf(ex * ex + ey * ey);
    float U = fmaxf(rad * rad, 1e-30f);
    if (!(U < INFINITY)) U = INFINITY;

    float lo = -1.f, hi = INFINITY;
    int cnt = -1;
    bool ok = false;
    if (k <= CAP) {
        for (int it = 0; it < MAX_REFINE; ++it) {
            int c = 0;
            const float Uc = U;
            visit_disk(p, cs, P, qx, qy, Uc, slack, [&](float d2, int idx) {
                if (d2 <= Uc) {
                    if (c < CAP) s_list[c * QUERY_THREADS + lane] = make_key(d2, idx);
                    ++c;
                }
            });
            cnt = c;
            if (cnt >= k && cnt <= CAP) { ok = true; break; }
            if (cnt < k) lo = U; else hi = U;
            float Un = U * target / fmaxf(float(cnt), 0.5f);
            Un = (cnt < k) ? fmaxf(Un, U * 1.25f) : fminf(Un, U * 0.8f);
            if (!(Un > lo && Un < hi)) Un = (hi < INFINITY) ? 0.5f * (fmaxf(lo, 0.f) + hi) : U * 4.f;
            if (!(Un > lo && Un < hi)) break;
            U = Un;
        }
    }

    if (ok) {
        uint64_t a[CAP];
#pragma unroll
        for (int s = 0; s < CAP; ++s) a[s] = (s < cnt) ? s_list[s * QUERY_THREADS + lane] : ~0ull;
        bitonic_sort<CAP>(a);
#pragma unroll
        for (int j = 0; j < CAP; ++j)
            if (j < k) store_result(out_idx, idx_i64, out_d2, obase + j, a[j]);
        return;
    }

    // Fallback: k exact passes, each taking the smallest key above the last.
    const float Uf = (hi < INFINITY) ? hi : INFINITY;
    uint64_t last = 0;
    for (int j = 0; j < k; ++j) {
        uint64_t best = ~0ull;
        const bool first = (j == 0);
        visit_disk(p, cs, P, qx, qy, Uf, slack, [&](float d2, int idx) {
            if (d2 <= Uf) {
                const uint64_t key = make_key(d2, idx);
                if ((first || key > last) && key < best) best = key;
            }
        });
        store_result(out_idx, idx_i64, out_d2, obase + j, best);
        last = best;
    }
}

}  // namespace knn
}  // namespace aff

using namespace aff;

extern "C" size_t aff_knn_workspace_bytes(int B, int M, int N, int D, int k) {
    (void)M; (void)D; (void)k;
    if (B <= 0 || N <= 0) return 0;
    return knn::ws_layout(B, N).total;
}

extern "C" aff_status aff_knn(const float *query, int64_t q_sb, int64_t q_sm, const float *ref,
                              int64_t r_sb, int64_t r_sn, int B, int M, int N, int D, int k,
                              void *out_idx, int idx_is_i64, float *out_d2, void *ws,
                              size_t ws_bytes, aff_stream_t stream) {
    AFF_CHECK_ARG(B >= 0 && M >= 0, "aff_knn: B=%d and M=%d must be >= 0", B, M);
    AFF_CHECK_ARG(N >= 1, "aff_knn: N=%d must be >= 1", N);
    AFF_CHECK_ARG(k >= 1 && k <= N, "aff_knn: k=%d exceeds number of reference points N=%d (or k < 1)", k, N);
    if (D != 2) return fail(AFF_ERR_UNSUPPORTED, "aff_knn: D=%d not supported (only D=2)", D);
    AFF_CHECK_ARG(q_sb >= 0 && q_sm >= 0 && r_sb >= 0 && r_sn >= 0, "aff_knn: negative stride");
    if (B == 0 || M == 0) return AFF_OK;
    AFF_CHECK_ARG(query && ref && out_idx, "aff_knn: NULL query/ref/out_idx");
    const knn::WsLayout L = knn::ws_layout(B, N);
    if (!ws || ws_bytes < L.total)
        return fail(AFF_ERR_WORKSPACE, "aff_knn: workspace of %zu bytes needed, got %zu", L.total, ws_bytes);
    AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(ws) & 255) == 0, "aff_knn: workspace must be 256-byte aligned");
    AFF_CHECK_ARG(B <= 65535, "aff_knn: B=%d exceeds 65535", B);

    hipStream_t s = static_cast<hipStream_t>(stream);
    char *w = static_cast<char *>(ws);
    auto *gp = reinterpret_cast<knn::GridParams *>(w + L.params);
    auto *cells = reinterpret_cast<int *>(w + L.cells);
    auto *pts = reinterpret_cast<float4 *>(w + L.pts);

    hipLaunchKernelGGL(knn::grid_build_kernel, dim3(B), dim3(knn::BUILD_THREADS), 0, s, ref, r_sb,
                       r_sn, N, L.cmax, gp, cells, pts);
    aff_status st = check_launch("aff_knn/grid_build");
    if (st != AFF_OK) return st;

    dim3 grid((M + knn::QUERY_THREADS - 1) / knn::QUERY_THREADS, B);
    dim3 block(knn::QUERY_THREADS);
    if (k <= 12)
        hipLaunchKernelGGL(knn::knn_query_kernel<16>, grid, block, 0, s, query, q_sb, q_sm, gp, cells,
                           pts, M, N, k, L.cmax, out_idx, idx_is_i64, out_d2);
    else if (k <= 24)
        hipLaunchKernelGGL(knn::knn_query_kernel<32>, grid, block, 0, s, query, q_sb, q_sm, gp, cells,
                           pts, M, N, k, L.cmax, out_idx, idx_is_i64, out_d2);
    else
        hipLaunchKernelGGL(knn::knn_query_kernel<64>, grid, block, 0, s, query, q_sb, q_sm, gp, cells,
                           pts, M, N, k, L.cmax, out_idx, idx_is_i64, out_d2);
    return check_launch("aff_knn/query");
}
