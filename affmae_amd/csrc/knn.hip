// Exact 2-D K-nearest-neighbour search for gfx950 (aff_knn) and the grid
// build shared with the deformable-attention kernels.
//
// Semantics follow the streaming top-K kernels of the reference
// (src/layers/kernels/knn.py:258-337, 422-471): squared Euclidean distance in
// fp32, results in ascending distance, equal distances resolved by the lower
// reference index.  The order is made explicit by sorting 64-bit keys, so it
// does not depend on visit order.
//
// Instead of streaming every reference point per query (O(M*N)), each image's
// reference points are counting-sorted into a uniform cell grid (one
// workgroup per image, histogram in LDS), and each query (one lane) visits
// only the cells that can hold points within a radius U, adjusted until the
// number of points with d2 <= U lies in [k, CAP]; those candidates are kept
// in a per-lane LDS column, sorted in registers by a bitonic network and the
// first k written (grid2d.hpp).  k > 64 streams k exact "next smallest key"
// passes over the cells.
#include "grid2d.hpp"

namespace aff {
namespace grid {

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

// One workgroup per segment (b, l): bounding box, ~n/2-cell uniform grid,
// LDS histogram, block scan, scatter into cell order.  The stored index of a
// point is its row within the batch item (s.start[l] + local index).
__global__ __launch_bounds__(BUILD_THREADS) void grid_build_kernel(const float *__restrict__ src, int64_t sb,
                                                                   int64_t sn, const Segs s, void *ws, WsLayout L) {
    __shared__ int s_cnt[MAX_CELLS];
    __shared__ float s_red[4][BUILD_THREADS / 64];
    __shared__ int s_wave[BUILD_THREADS / 64];
    __shared__ GridParams s_gp;

    const int seg = blockIdx.x;
    const int b = seg / s.L, l = seg % s.L;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    constexpr int NW = BUILD_THREADS / 64;
    const int n = s.start[l + 1] - s.start[l];
    const int cmax = s.cmax[l];
    const float *R = src + (int64_t)b * sb + (int64_t)s.start[l] * sn;
    char *w = static_cast<char *>(ws);
    GridParams *gp_out = reinterpret_cast<GridParams *>(w + L.params) + seg;
    int *cells = reinterpret_cast<int *>(w + L.cells) + (int64_t)b * s.cells_per_b + s.cell_off[l];
    float4 *pts = reinterpret_cast<float4 *>(w + L.pts) + (int64_t)b * s.npts_b + s.start[l];

    // 1. bounding box
    float xmn = INFINITY, xmx = -INFINITY, ymn = INFINITY, ymx = -INFINITY;
    for (int i = tid; i < n; i += BUILD_THREADS) {
        float x = R[(int64_t)i * sn], y = R[(int64_t)i * sn + 1];
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
        for (int q = 1; q < NW; ++q) {
            xmn = fminf(xmn, s_red[0][q]); xmx = fmaxf(xmx, s_red[1][q]);
            ymn = fminf(ymn, s_red[2][q]); ymx = fmaxf(ymx, s_red[3][q]);
        }
        GridParams p;
        p.x0 = xmn; p.y0 = ymn; p.pad = 0;
        const float wd = xmx - xmn, ht = ymx - ymn;
        const float ext = fmaxf(wd, ht);
        int gx = 1, gy = 1;
        float h = 1.f;
        if (ext > 0.f && ext < INFINITY) {
            const float T = float(cmax);
            const float wa = fmaxf(wd, ext / T), ha = fmaxf(ht, ext / T);
            h = sqrtf(wa * ha / T);
            for (;;) {
                gx = (int)fminf(wd / h + 1.f, T);
                gy = (int)fminf(ht / h + 1.f, T);
                if ((int64_t)gx * gy <= cmax) break;
                h *= 1.0625f;
            }
        } else {
            if (!(xmn > -INFINITY && xmn < INFINITY)) p.x0 = 0.f;
            if (!(ymn > -INFINITY && ymn < INFINITY)) p.y0 = 0.f;
        }
        p.h = h; p.inv_h = 1.f / h; p.gx = gx; p.gy = gy; p.ncell = gx * gy;
        s_gp = p;
        *gp_out = p;
    }
    __syncthreads();
    const GridParams p = s_gp;
    const int ncell = p.ncell;

    // 3. histogram
    for (int c = tid; c < ncell; c += BUILD_THREADS) s_cnt[c] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += BUILD_THREADS) {
        float x = R[(int64_t)i * sn], y = R[(int64_t)i * sn + 1];
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
    for (int c = c0; c < c1; ++c) {
        int cnt = s_cnt[c];
        cells[c] = run;
        s_cnt[c] = run;  // becomes the scatter cursor
        run += cnt;
    }
    if (tid == 0) cells[ncell] = n;
    __syncthreads();

    // 5. scatter points into cell order
    for (int i = tid; i < n; i += BUILD_THREADS) {
        float x = R[(int64_t)i * sn], y = R[(int64_t)i * sn + 1];
        int c = cell_coord(y, p.y0, p.inv_h, p.gy) * p.gx + cell_coord(x, p.x0, p.inv_h, p.gx);
        int slot = atomicAdd(&s_cnt[c], 1);
        pts[slot] = make_float4(x, y, __int_as_float(s.start[l] + i), 0.f);
    }
}

aff_status launch_build(const float *src, int64_t sb, int64_t sn, int B, const Segs &s, void *ws,
                        hipStream_t stream) {
    const WsLayout L = ws_layout(B, s);
    hipLaunchKernelGGL(grid_build_kernel, dim3(B * s.L), dim3(BUILD_THREADS), 0, stream, src, sb, sn, s, ws, L);
    return check_launch("grid_build");
}

}  // namespace grid

namespace knn {

using namespace grid;
constexpr int QUERY_THREADS = 64;

__device__ __forceinline__ void store_result(void *out_idx, int idx_i64, float *out_d2, int64_t o, uint64_t key) {
    const int idx = key_index(key);
    if (idx_i64)
        static_cast<int64_t *>(out_idx)[o] = idx;
    else
        static_cast<int32_t *>(out_idx)[o] = idx;
    if (out_d2) out_d2[o] = key_d2(key);
}

template <int CAP>
__global__ __launch_bounds__(QUERY_THREADS) void knn_query_kernel(const float *__restrict__ query, int64_t q_sb,
                                                                  int64_t q_sm, const Segs s, const void *ws,
                                                                  WsLayout L, int M, int k, void *__restrict__ out_idx,
                                                                  int idx_i64, float *__restrict__ out_d2) {
    __shared__ uint64_t s_list[CAP * QUERY_THREADS];
    const int lane = threadIdx.x;
    const int b = blockIdx.y;
    const int qi = blockIdx.x * QUERY_THREADS + lane;
    if (qi >= M) return;
    const SegView g = seg_view(ws, L, s, b, 0);
    const float *Q = query + (int64_t)b * q_sb + (int64_t)qi * q_sm;
    const float qx = Q[0], qy = Q[1];
    const int64_t obase = ((int64_t)b * M + qi) * k;

    if (k <= CAP) {
        uint64_t a[CAP];
        knn_select<CAP>(g, qx, qy, k, s_list + lane, QUERY_THREADS, a);
#pragma unroll
        for (int j = 0; j < CAP; ++j)
            if (j < k) store_result(out_idx, idx_i64, out_d2, obase + j, a[j]);
        return;
    }
    // k > CAP: k exact passes over every cell, each taking the smallest key
    // above the previous one.
    const float slack = query_slack(g.p, qx, qy);
    uint64_t last = 0;
    for (int j = 0; j < k; ++j) {
        uint64_t best = ~0ull;
        const bool first = (j == 0);
        visit_disk(g, qx, qy, INFINITY, slack, [&](float d2, int idx) {
            const uint64_t key = make_key(d2, idx);
            if ((first || key > last) && key < best) best = key;
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
    const grid::Segs s = grid::make_segs(1, &N);
    return grid::ws_layout(B, s).total;
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
    const grid::Segs s = grid::make_segs(1, &N);
    const grid::WsLayout L = grid::ws_layout(B, s);
    if (!ws || ws_bytes < L.total)
        return fail(AFF_ERR_WORKSPACE, "aff_knn: workspace of %zu bytes needed, got %zu", L.total, ws_bytes);
    AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(ws) & 255) == 0, "aff_knn: workspace must be 256-byte aligned");
    AFF_CHECK_ARG(B <= 65535, "aff_knn: B=%d exceeds 65535", B);

    hipStream_t st = static_cast<hipStream_t>(stream);
    aff_status r = grid::launch_build(ref, r_sb, r_sn, B, s, ws, st);
    if (r != AFF_OK) return r;
    dim3 gridd((M + knn::QUERY_THREADS - 1) / knn::QUERY_THREADS, B);
    dim3 block(knn::QUERY_THREADS);
    if (k <= 12)
        hipLaunchKernelGGL(knn::knn_query_kernel<16>, gridd, block, 0, st, query, q_sb, q_sm, s, ws, L, M, k, out_idx,
                           idx_is_i64, out_d2);
    else if (k <= 24)
        hipLaunchKernelGGL(knn::knn_query_kernel<32>, gridd, block, 0, st, query, q_sb, q_sm, s, ws, L, M, k, out_idx,
                           idx_is_i64, out_d2);
    else
        hipLaunchKernelGGL(knn::knn_query_kernel<64>, gridd, block, 0, st, query, q_sb, q_sm, s, ws, L, M, k, out_idx,
                           idx_is_i64, out_d2);
    return check_launch("aff_knn/query");
}
