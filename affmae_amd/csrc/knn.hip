// Exact 2-D K-nearest-neighbour search for gfx950 (aff_knn) and the grid
// build shared with the deformable-attention kernels.
//
// Semantics follow the streaming top-K kernels of the reference
// (src/layers/kernels/knn.py:258-337, 422-471): squared Euclidean distance in
// fp32, results in ascending distance, equal distances resolved by the lower
// reference index.  The order is made explicit by sorting 64-bit keys
// (d2 bits, index), so it does not depend on visit order.
//
// Instead of streaming every reference point per query (O(M*N)), each image's
// reference points are counting-sorted into a uniform cell grid (one
// workgroup per image, histogram in LDS).  The same workgroup sorts the
// queries by square cell tile of that grid (sized for ~48 queries, tiles in
// serpentine order), so 64 consecutive sorted queries cover a compact patch.
//
// knn_win_kernel: one wave per 64 sorted queries.  The wave copies the cells
// around its patch (the union of the lanes' search disks) into LDS with
// coalesced loads, then every lane runs its own exact search against the LDS
// copy: from a local-density estimate it picks a radius U, visits the cells
// whose rows meet the disk d2 <= U, and adjusts U until the number of points
// inside lies in [k, CAP].  Candidates are kept as 16-bit window slots in a
// per-lane LDS column, turned into keys, sorted in registers by a sorting
// network, and the first k written.  A lane whose disk leaves the window (or
// whose radius search cannot isolate k points because of exact distance
// ties) redoes its query against the global grid; exact ties then take k
// "next smallest key" passes.  knn_query_kernel (one lane per query, global
// grid only) serves k > 64 and images of more than 65536 points.
#include "grid2d.hpp"
#include "knn_brute.hpp"

#include <limits.h>

#include <mutex>

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

// In-place exclusive scan of s_cnt[0, n) by BUILD_THREADS threads (each owns a
// contiguous chunk); the offsets are also written to gout[0, n] when gout is
// non-null (gout[n] = total).  Ends with a barrier.
__device__ void block_exclusive_scan(int *s_cnt, int n, int *s_wave, int *gout) {
    constexpr int NW = BUILD_THREADS / 64;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int chunk = (n + BUILD_THREADS - 1) / BUILD_THREADS;
    const int c0 = min(tid * chunk, n), c1 = min(c0 + chunk, n);
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
        const int cnt = s_cnt[c];
        if (gout) gout[c] = run;
        s_cnt[c] = run;  // becomes the scatter cursor
        run += cnt;
    }
    if (gout && tid == BUILD_THREADS - 1) gout[n] = run;
    __syncthreads();
}

// One workgroup per segment (b, l): bounding box, ~n/2-cell uniform grid,
// LDS histogram, block scan, scatter into cell order.  The stored index of a
// point is its row within the batch item (s.start[l] + local index).  With
// qb.out set (single-segment grids), the queries are then counting-sorted by
// cell tile into qb.out[b * M + slot] = (x, y, query index bits, 0).
__global__ __launch_bounds__(BUILD_THREADS) void grid_build_kernel(const float *__restrict__ src, int64_t sb,
                                                                   int64_t sn, const Segs s, void *ws, WsLayout L,
                                                                   QueryBin qb, ZeroSpan z) {
    __shared__ int s_cnt[MAX_CELLS];
    __shared__ float s_red[4][BUILD_THREADS / 64];
    __shared__ int s_wave[BUILD_THREADS / 64];
    __shared__ GridParams s_gp;

    const int seg = blockIdx.x;
    const int b = seg / s.L, l = seg % s.L;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    if (seg == 0)
        for (int i = tid; i < z.n; i += BUILD_THREADS) z.p[i] = 0;
    constexpr int NW = BUILD_THREADS / 64;
    const int n = s.start[l + 1] - s.start[l];
    const int cmax = s.cmax[l];
    const float *R = src + (int64_t)b * sb + (int64_t)s.start[l] * sn;
    char *w = static_cast<char *>(ws);
    GridParams *gp_out = reinterpret_cast<GridParams *>(w + L.params) + seg;
    int *cells = reinterpret_cast<int *>(w + L.cells) + (int64_t)b * s.cells_per_b + s.cell_off[l];
    float4 *pts = reinterpret_cast<float4 *>(w + L.pts) + (int64_t)b * s.npts_b + s.start[l];

    // Points i = tid + j * BUILD_THREADS, j < PPT, are read once into
    // registers; larger segments re-read the rest from global memory.
    float rx[PPT], ry[PPT];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int i = tid + j * BUILD_THREADS;
        rx[j] = ry[j] = 0.f;
        if (i < n) {
            rx[j] = R[(int64_t)i * sn];
            ry[j] = R[(int64_t)i * sn + 1];
        }
    }

    // 1. bounding box
    float xmn = INFINITY, xmx = -INFINITY, ymn = INFINITY, ymx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PPT; ++j)
        if (tid + j * BUILD_THREADS < n) {
            xmn = fminf(xmn, rx[j]); xmx = fmaxf(xmx, rx[j]);
            ymn = fminf(ymn, ry[j]); ymx = fmaxf(ymx, ry[j]);
        }
    for (int i = tid + PPT * BUILD_THREADS; i < n; i += BUILD_THREADS) {
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
    auto cell_of = [&](float x, float y) {
        return cell_coord(y, p.y0, p.inv_h, p.gy) * p.gx + cell_coord(x, p.x0, p.inv_h, p.gx);
    };
    int cl[PPT];  // each point's cell, for both passes
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        cl[j] = cell_of(rx[j], ry[j]);
        if (tid + j * BUILD_THREADS < n) atomicAdd(&s_cnt[cl[j]], 1);
    }
    for (int i = tid + PPT * BUILD_THREADS; i < n; i += BUILD_THREADS)
        atomicAdd(&s_cnt[cell_of(R[(int64_t)i * sn], R[(int64_t)i * sn + 1])], 1);
    __syncthreads();

    // 4. exclusive scan -> cell offsets
    block_exclusive_scan(s_cnt, ncell, s_wave, cells);

    // 5. scatter points into cell order
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int i = tid + j * BUILD_THREADS;
        if (i < n) {
            const int slot = atomicAdd(&s_cnt[cl[j]], 1);
            pts[slot] = make_float4(rx[j], ry[j], __int_as_float(s.start[l] + i), 0.f);
        }
    }
    for (int i = tid + PPT * BUILD_THREADS; i < n; i += BUILD_THREADS) {
        const float x = R[(int64_t)i * sn], y = R[(int64_t)i * sn + 1];
        const int slot = atomicAdd(&s_cnt[cell_of(x, y)], 1);
        pts[slot] = make_float4(x, y, __int_as_float(s.start[l] + i), 0.f);
    }
    if (qb.out == nullptr) return;

    // 6. queries by tile of this grid: square T x T cell tiles holding about
    // qb.tile_queries queries each, visited in serpentine order (tile rows
    // alternate direction), so consecutive tiles always touch
    __syncthreads();
    const int M = qb.M;
    const float *Q = qb.q + (int64_t)b * qb.q_sb;
    // the queries are the reference points (same array): reuse the registers
    const bool same = Q == R && qb.q_sm == sn && M == n;
    float qx[PPT], qy[PPT];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int i = tid + j * BUILD_THREADS;
        qx[j] = rx[j];
        qy[j] = ry[j];
        if (!same && i < M) {
            qx[j] = Q[(int64_t)i * qb.q_sm];
            qy[j] = Q[(int64_t)i * qb.q_sm + 1];
        }
    }
    const int tq = qb.tile_queries > 0 ? qb.tile_queries : TILE_QUERIES;
    const int T = max(1, (int)rintf(sqrtf(float(tq) * float(ncell) / float(max(M, 1)))));
    const int ntx = (p.gx + T - 1) / T, nty = (p.gy + T - 1) / T;
    const int ntile = ntx * nty;
    // c / T for 0 <= c < 2^24 without an integer division: a float quotient,
    // corrected by one either way
    const float inv_t = 1.f / float(T);
    auto div_t = [&](int c) {
        int d = int(float(c) * inv_t);
        d -= d * T > c ? 1 : 0;
        d += (d + 1) * T <= c ? 1 : 0;
        return d;
    };
    auto tile_of = [&](float x, float y) {
        const int tx = div_t(cell_coord(x, p.x0, p.inv_h, p.gx)), ty = div_t(cell_coord(y, p.y0, p.inv_h, p.gy));
        return ty * ntx + ((ty & 1) ? ntx - 1 - tx : tx);
    };
    for (int c = tid; c < ntile; c += BUILD_THREADS) s_cnt[c] = 0;
    __syncthreads();
    int tl[PPT];  // each query's tile, for both passes
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        tl[j] = tile_of(qx[j], qy[j]);
        if (tid + j * BUILD_THREADS < M) atomicAdd(&s_cnt[tl[j]], 1);
    }
    for (int i = tid + PPT * BUILD_THREADS; i < M; i += BUILD_THREADS)
        atomicAdd(&s_cnt[tile_of(Q[(int64_t)i * qb.q_sm], Q[(int64_t)i * qb.q_sm + 1])], 1);
    __syncthreads();
    block_exclusive_scan(s_cnt, ntile, s_wave, nullptr);
    float4 *qo = qb.out + (int64_t)b * M;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int i = tid + j * BUILD_THREADS;
        if (i < M) qo[atomicAdd(&s_cnt[tl[j]], 1)] = make_float4(qx[j], qy[j], __int_as_float(i), 0.f);
    }
    for (int i = tid + PPT * BUILD_THREADS; i < M; i += BUILD_THREADS) {
        const float x = Q[(int64_t)i * qb.q_sm], y = Q[(int64_t)i * qb.q_sm + 1];
        qo[atomicAdd(&s_cnt[tile_of(x, y)], 1)] = make_float4(x, y, __int_as_float(i), 0.f);
    }
}

static aff_status launch_build_impl(const float *src, int64_t sb, int64_t sn, int B, const Segs &s, void *ws,
                                    hipStream_t stream, const QueryBin &qb, const ZeroSpan &z) {
    const WsLayout L = ws_layout(B, s);
    hipLaunchKernelGGL(grid_build_kernel, dim3(B * s.L), dim3(BUILD_THREADS), 0, stream, src, sb, sn, s, ws, L, qb,
                       z);
    return check_launch("grid_build");
}

aff_status launch_build(const float *src, int64_t sb, int64_t sn, int B, const Segs &s, void *ws,
                        hipStream_t stream, const QueryBin &qb) {
    return launch_build_impl(src, sb, sn, B, s, ws, stream, qb, ZeroSpan{nullptr, 0});
}

aff_status launch_build(const float *src, int64_t sb, int64_t sn, int B, const Segs &s, void *ws,
                        hipStream_t stream, const ZeroSpan &z) {
    return launch_build_impl(src, sb, sn, B, s, ws, stream, QueryBin{nullptr, 0, 0, 0, nullptr, 0}, z);
}

aff_status launch_build(const float *src, int64_t sb, int64_t sn, int B, const Segs &s, void *ws,
                        hipStream_t stream) {
    return launch_build(src, sb, sn, B, s, ws, stream, QueryBin{nullptr, 0, 0, 0, nullptr, 0});
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

// The first k sorted keys of one query: one loop per output array, so each
// store is a fixed base plus an immediate offset.
template <int CAP>
__device__ __forceinline__ void store_row(const uint64_t (&a)[CAP], int k, void *out_idx, int idx_i64, float *out_d2,
                                          int64_t obase) {
    if (idx_i64) {
        int64_t *o = static_cast<int64_t *>(out_idx) + obase;
#pragma unroll
        for (int j = 0; j < CAP; ++j)
            if (j < k) o[j] = key_index(a[j]);
    } else {
        int32_t *o = static_cast<int32_t *>(out_idx) + obase;
#pragma unroll
        for (int j = 0; j < CAP; ++j)
            if (j < k) o[j] = key_index(a[j]);
    }
    if (out_d2) {
        float *o = out_d2 + obase;
#pragma unroll
        for (int j = 0; j < CAP; ++j)
            if (j < k) o[j] = key_d2(a[j]);
    }
}

// One lane per query against the global grid: k > 64 (k exact passes) and
// the general path for images larger than the windowed kernel takes.
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

// ------------------------------------------------------- windowed kernel --
constexpr int WIN_THREADS = 64;
constexpr int WMAX = 640;       // window points held in LDS (queries as dense as the points)
constexpr int WMAX_WIDE = 1024; // the same for sparser queries (M < N / 2): wider windows
constexpr int WCMAX = 320;      // window cell-offset entries, (WX + 1) * WY
constexpr int WCMAX_WIDE = 640; // the same for the wide window
constexpr int WROWS = 64;       // window rows (one lane each while sizing)
constexpr float WIN_U = 1.6f;   // window disk: radius^2 = WIN_U * the initial estimate
constexpr int MAX_SLOT = 65536; // 16-bit candidate slots

// Per-lane candidate column of 16-bit slots: entry c of lane `lane` is
// halfword c * 64 + lane of the list, so consecutive entries of a lane are
// 128 bytes apart and a wave's 64 stores fill 128 contiguous bytes.
__device__ __forceinline__ void list_put(uint32_t *lst, int c, int lane, int v) {
    reinterpret_cast<uint16_t *>(lst)[c * WIN_THREADS + lane] = uint16_t(v);
}
__device__ __forceinline__ int list_get(const uint32_t *lst, int c, int lane) {
    return reinterpret_cast<const uint16_t *>(lst)[c * WIN_THREADS + lane];
}

struct Window {
    const float2 *xy;  // LDS points (window slot order)
    const int *wcs;    // LDS slot of the first point of window cell (r, c), c in [0, WX]
    int wx0, wy0, wx1, wy1, wx1p;  // wx1p = WX + 1
};

// Visits the window points of every cell meeting the disk d2 <= U (the same
// cell set visit_disk() takes), calling f(d2, window slot, valid) in groups
// of four (valid == false pads a row's last group).  Returns false when that
// cell set reaches beyond the window.  The chord bounds use the hardware
// square root (1 ulp); the slack term dominates its error, so the visited
// set is still a superset.
template <typename F>
__device__ __forceinline__ bool visit_disk_win(const GridParams &p, const Window &w, float qx, float qy, float U,
                                               float slack, F &&f) {
    const float r = __builtin_amdgcn_sqrtf(U) * 1.00002f + slack;
    const int cy0 = cell_coord(qy - r, p.y0, p.inv_h, p.gy);
    const int cy1 = cell_coord(qy + r, p.y0, p.inv_h, p.gy);
    bool covered = cy0 >= w.wy0 && cy1 <= w.wy1;
    const int ya = max(cy0, w.wy0), yb = min(cy1, w.wy1);
    for (int cy = ya; cy <= yb; ++cy) {
        const float rlo = p.y0 + float(cy) * p.h, rhi = rlo + p.h;
        const float dy = fmaxf(0.f, fmaxf(rlo - qy, qy - rhi) - slack);
        const float w2 = r * r - dy * dy;
        if (!(w2 >= 0.f)) continue;
        const float hw = __builtin_amdgcn_sqrtf(w2) * 1.00002f + slack;
        const int cx0 = cell_coord(qx - hw, p.x0, p.inv_h, p.gx);
        const int cx1 = cell_coord(qx + hw, p.x0, p.inv_h, p.gx);
        covered = covered && cx0 >= w.wx0 && cx1 <= w.wx1;
        const int xa = max(cx0, w.wx0), xb = min(cx1, w.wx1);
        if (xa > xb) continue;
        const int *row = w.wcs + (cy - w.wy0) * w.wx1p - w.wx0;
        const int beg = row[xa], end = row[xb + 1];
        for (int t = beg; t < end; t += 4) {
            float2 pt[4];  // the window array has 3 spare entries past its end
#pragma unroll
            for (int u = 0; u < 4; ++u) pt[u] = w.xy[t + u];
#pragma unroll
            for (int u = 0; u < 4; ++u) f(dist2(pt[u].x, pt[u].y, qx, qy), t + u, t + u < end);
        }
    }
    return covered;
}

// The starting radius^2 of a lane's window search: u scaled so that the
// expected number of points in the disk is `target`.  The expectation sums,
// over the grid rows whose centre line meets the disk, the points of the cells
// the chord along that line spans, end cells in proportion to their covered
// width (cell counts from the window's cell table).  Returns u unchanged when
// the disk reaches outside the window.  Only the number of refinement passes
// depends on it: every pass still counts exactly.
__device__ __forceinline__ float window_radius2(const GridParams &p, const Window &w, float qx, float qy, float u,
                                               float target) {
    const float rad = __builtin_amdgcn_sqrtf(u);
    const int cy0 = cell_coord(qy - rad, p.y0, p.inv_h, p.gy), cy1 = cell_coord(qy + rad, p.y0, p.inv_h, p.gy);
    if (cy0 < w.wy0 || cy1 > w.wy1) return u;
    float est = 0.f;
    bool inside = true;
    for (int cy = cy0; cy <= cy1; ++cy) {
        const float dy = p.y0 + (float(cy) + 0.5f) * p.h - qy;
        const float w2 = u - dy * dy;
        if (!(w2 > 0.f)) continue;
        const float hw = __builtin_amdgcn_sqrtf(w2);
        const float xa = qx - hw, xb = qx + hw;
        const int ca = cell_coord(xa, p.x0, p.inv_h, p.gx), cb = cell_coord(xb, p.x0, p.inv_h, p.gx);
        inside = inside && ca >= w.wx0 && cb <= w.wx1;
        const int *row = w.wcs + (cy - w.wy0) * w.wx1p - w.wx0;
        const int ia = min(max(ca, w.wx0), w.wx1), ib = min(max(cb, w.wx0), w.wx1);
        const float na = float(row[ia + 1] - row[ia]), nb = float(row[ib + 1] - row[ib]);
        // uncovered fractions of the end cells
        const float fa = fminf(fmaxf((xa - (p.x0 + float(ia) * p.h)) * p.inv_h, 0.f), 1.f);
        const float fb = fminf(fmaxf((p.x0 + float(ib + 1) * p.h - xb) * p.inv_h, 0.f), 1.f);
        est += float(row[ib + 1] - row[ia]) - fa * na - fb * nb;
    }
    return inside ? u * target / fmaxf(est, 1.f) : u;
}

// visit_disk() reporting the point's slot in the cell-ordered array too:
// f(d2, slot, index).
template <typename F>
__device__ __forceinline__ void visit_disk_slots(const SegView &g, float qx, float qy, float U, float slack, F &&f) {
    const GridParams &p = g.p;
    const float r = sqrtf(U) * 1.00002f + slack;
    const int cy0 = cell_coord(qy - r, p.y0, p.inv_h, p.gy);
    const int cy1 = cell_coord(qy + r, p.y0, p.inv_h, p.gy);
    for (int cy = cy0; cy <= cy1; ++cy) {
        const float rlo = p.y0 + float(cy) * p.h, rhi = rlo + p.h;
        const float dy = fmaxf(0.f, fmaxf(rlo - qy, qy - rhi) - slack);
        const float w2 = r * r - dy * dy;
        if (!(w2 >= 0.f)) continue;
        const float hw = sqrtf(w2) + slack;
        const int cx0 = cell_coord(qx - hw, p.x0, p.inv_h, p.gx);
        const int cx1 = cell_coord(qx + hw, p.x0, p.inv_h, p.gx);
        const int beg = g.cs[cy * p.gx + cx0], end = g.cs[cy * p.gx + cx1 + 1];
        for (int t = beg; t < end; t += 4) {  // four loads in flight per step
            float4 pt[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) pt[u] = g.P[min(t + u, end - 1)];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (t + u < end) f(dist2(pt[u].x, pt[u].y, qx, qy), t + u, __float_as_int(pt[u].z));
        }
    }
}

// Radius search shared by the window and global sources: returns the
// number of candidates (in [k, CAP]) written to the lane's column, or -1
// when the source cannot settle it (window left, or ties).
// Appends go to entry min(c, CAP), or to the spare entry CAP + 1 when the
// point is outside the disk, so the store is unconditional (no branch).
template <int CAP, typename Visit>
__device__ __forceinline__ int radius_select(Visit &&visit, float U, int k, uint32_t *lst, int lane, float &hi_out) {
    const float target = 0.5f * float(k + CAP);
    float lo = -1.f, hi = INFINITY;
    for (int it = 0; it < MAX_REFINE; ++it) {
        int c = 0;
        const float Uc = U;
        const bool ok = visit(Uc, [&](float d2, int slot, bool valid) {
            const bool in = valid && d2 <= Uc;
            list_put(lst, in ? min(c, CAP) : CAP + 1, lane, slot);
            c += in ? 1 : 0;
        });
        if (!ok) return -1;
        if (c >= k && c <= CAP) return c;
        if (c < k) lo = U; else hi = U;
        float Un = U * target / fmaxf(float(c), 0.5f);
        Un = (c < k) ? fmaxf(Un, U * 1.25f) : fminf(Un, U * 0.8f);
        if (!(Un > lo && Un < hi)) Un = (hi < INFINITY) ? 0.5f * (fmaxf(lo, 0.f) + hi) : U * 4.f;
        if (!(Un > lo && Un < hi)) break;
        U = Un;
    }
    hi_out = hi;
    return -1;
}

// The first k sorted keys of the wave's queries, written row by row: the keys
// go through LDS (buf: (CAP / 2 + 1) words per lane) in column chunks of CAP / 2,
// and each store instruction then covers consecutive words of a few output rows
// instead of one word in each of 64 rows.  qrow[r] is the output row of lane r;
// rows r >= nq are not written.  Called by the whole wave.
template <int CAP>
__device__ __forceinline__ void store_rows_wave(const uint64_t (&a)[CAP], int k, int nq, const int *qrow,
                                                uint32_t *buf, int lane, void *out_idx, int idx_i64, float *out_d2,
                                                int64_t row0) {
    constexpr int CW = CAP / 2, SP = CW + 1;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1 && !out_d2) break;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int c0 = h * CW;
            if (c0 >= k) break;
            const int cols = min(CW, k - c0);
            __syncthreads();  // the buffer's previous readers are done
#pragma unroll
            for (int j = 0; j < CW; ++j)
                if (j < cols) buf[lane * SP + j] = pass ? uint32_t(a[c0 + j] >> 32) : uint32_t(a[c0 + j]);
            __syncthreads();
            const int rpi = WIN_THREADS / cols;  // rows per store instruction
            const int rr = lane / cols, c = lane - rr * cols;
            // eight store instructions per step, their LDS reads issued together
            for (int r0 = 0; r0 < nq; r0 += 8 * rpi) {
                uint32_t v[8];
                int64_t o[8];
                bool ok[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int r = r0 + u * rpi + rr;
                    ok[u] = rr < rpi && r < nq;
                    const int rc = ok[u] ? r : 0;
                    v[u] = buf[rc * SP + c];
                    o[u] = (row0 + qrow[rc]) * k + c0 + c;
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if (!ok[u]) continue;
                    if (pass) out_d2[o[u]] = __uint_as_float(v[u]);
                    else if (idx_i64) static_cast<int64_t *>(out_idx)[o[u]] = int32_t(v[u]);
                    else static_cast<int32_t *>(out_idx)[o[u]] = int32_t(v[u]);
                }
            }
        }
    }
}

template <int CAP, int WM, int WC, bool ROWS>
__global__ __launch_bounds__(WIN_THREADS) void knn_win_kernel(const float4 *__restrict__ qsorted, const Segs s,
                                                              const void *ws, WsLayout L, int M, int k,
                                                              void *__restrict__ out_idx, int idx_i64,
                                                              float *__restrict__ out_d2) {
    __shared__ float2 s_xy[WM + 3];  // + spare entries read (and ignored) by the 4-wide visits
    __shared__ uint16_t s_id[WM];  // point indices (the windowed path takes N <= 65536)
    __shared__ int s_wcs[WC];
    __shared__ int s_rb[WROWS + 1];
    __shared__ int s_gb[WROWS];
    __shared__ uint8_t s_rowof[WM];  // window row of each window point slot
    __shared__ uint32_t s_list[(CAP / 2 + 1) * WIN_THREADS];  // CAP entries + 2 spare entries per lane

    const int lane = threadIdx.x;
    const int b = blockIdx.y;
    const int i = blockIdx.x * WIN_THREADS + lane;
    const bool active = i < M;
    const float4 qp = qsorted[(int64_t)b * M + min(i, M - 1)];
    const float qx = qp.x, qy = qp.y;
    const int qi = __float_as_int(qp.z);
    const SegView g = seg_view(ws, L, s, b, 0);
    const GridParams &p = g.p;
    const float slack = query_slack(p, qx, qy);
    const float U0 = initial_radius2(g, qx, qy, 0.5f * float(k + CAP));

    // ---- window: cells meeting the union of the lanes' disks of radius^2 WIN_U * U0
    int wx0, wx1, wy0, wy1;
    {
        const float rw = sqrtf(U0 * WIN_U) * 1.00002f + slack;
        int cx0 = cell_coord(qx - rw, p.x0, p.inv_h, p.gx), cx1 = cell_coord(qx + rw, p.x0, p.inv_h, p.gx);
        int cy0 = cell_coord(qy - rw, p.y0, p.inv_h, p.gy), cy1 = cell_coord(qy + rw, p.y0, p.inv_h, p.gy);
        if (!active) { cx0 = cy0 = INT_MAX; cx1 = cy1 = INT_MIN; }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            cx0 = min(cx0, __shfl_xor(cx0, o, 64));
            cy0 = min(cy0, __shfl_xor(cy0, o, 64));
            cx1 = max(cx1, __shfl_xor(cx1, o, 64));
            cy1 = max(cy1, __shfl_xor(cy1, o, 64));
        }
        wx0 = cx0; wx1 = cx1; wy0 = cy0; wy1 = cy1;
    }
    const int WX = wx1 - wx0 + 1, WY = wy1 - wy0 + 1;
    bool win = WY <= WROWS && (WX + 1) * WY <= WC;
    if (win) {
        int gb = 0, cnt = 0;
        if (lane < WY) {
            const int *row = g.cs + (wy0 + lane) * p.gx;
            gb = row[wx0];
            cnt = row[wx1 + 1] - gb;
        }
        int incl = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o, 64);
            if (lane >= o) incl += y;
        }
        const int total = __shfl(incl, 63, 64);
        win = total <= WM;
        if (win) {
            if (lane < WY) {
                s_rb[lane] = incl - cnt;
                s_gb[lane] = gb;
                for (int j = incl - cnt; j < incl; ++j) s_rowof[j] = uint8_t(lane);  // this row's slots
            }
            if (lane == 0) s_rb[WY] = total;
            __syncthreads();
            // cell table and points: each lane's loads are issued together, then
            // written, so the copy costs one memory round trip, not one per entry
            constexpr int WCI = (WC + WIN_THREADS - 1) / WIN_THREADS;
            const int ne = (WX + 1) * WY;
            int cv[WCI];
#pragma unroll
            for (int u = 0; u < WCI; ++u) {
                const int e = min(lane + u * WIN_THREADS, ne - 1);
                const int r = e / (WX + 1), c = e - r * (WX + 1);
                cv[u] = g.cs[(wy0 + r) * p.gx + wx0 + c];
            }
#pragma unroll
            for (int u = 0; u < WCI; ++u) {
                const int e = lane + u * WIN_THREADS;
                if (e < ne) {
                    const int r = e / (WX + 1);
                    s_wcs[e] = s_rb[r] + cv[u] - s_gb[r];
                }
            }
            constexpr int PB = 8;  // points per lane in flight
            for (int t0 = 0; t0 < total; t0 += PB * WIN_THREADS) {
                float4 pt[PB];
#pragma unroll
                for (int u = 0; u < PB; ++u) {
                    const int t = min(t0 + u * WIN_THREADS + lane, total - 1);
                    const int r = s_rowof[t];
                    pt[u] = g.P[s_gb[r] + (t - s_rb[r])];
                }
#pragma unroll
                for (int u = 0; u < PB; ++u) {
                    const int t = t0 + u * WIN_THREADS + lane;
                    if (t < total) {
                        s_xy[t] = make_float2(pt[u].x, pt[u].y);
                        s_id[t] = uint16_t(__float_as_int(pt[u].z));
                    }
                }
            }
            __syncthreads();
        }
    }

    // ---- per-lane exact search: window first, the global grid if needed
    float hi = INFINITY;
    int cnt = -1;
    bool from_win = false;
    if (active && win) {
        const Window w{s_xy, s_wcs, wx0, wy0, wx1, wy1, WX + 1};
        // (more waves than fit at once: total work counts, and the refined start saves
        // a wave most of a radius pass; in one resident generation it only adds latency)
        const float Uw = ROWS ? window_radius2(p, w, qx, qy, U0, 0.5f * float(k + CAP)) : U0;
        cnt = radius_select<CAP>(
            [&](float U, auto &&f) { return visit_disk_win(p, w, qx, qy, U, slack, f); }, Uw, k, s_list, lane, hi);
        from_win = cnt >= 0;
    }
    if (active && cnt < 0) {
        hi = INFINITY;
        cnt = radius_select<CAP>(
            [&](float U, auto &&f) {
                visit_disk_slots(g, qx, qy, U, slack, [&](float d2, int t, int idx) { (void)idx; f(d2, t, true); });
                return true;
            },
            U0, k, s_list, lane, hi);
        if (cnt < 0) {
            // exact ties at one distance: k passes, each taking the smallest
            // key above the previous one, inside the smallest disk that held
            // more than CAP points
            uint64_t last = 0;
            for (int j = 0; j < k; ++j) {
                uint64_t best = ~0ull;
                int bslot = 0;
                const bool first = (j == 0);
                visit_disk_slots(g, qx, qy, hi, slack, [&](float d2, int t, int idx) {
                    if (d2 <= hi) {
                        const uint64_t key = make_key(d2, idx);
                        if ((first || key > last) && key < best) {
                            best = key;
                            bslot = t;
                        }
                    }
                });
                list_put(s_list, j, lane, bslot);
                last = best;
            }
            cnt = k;
        }
    }
    // ---- keys, sort, first k out (inactive lanes carry keys ~0 and write nothing)
    // (loads fenced in groups of 8 so the scheduler does not hoist all of them
    // and raise the register count past two waves per SIMD)
    uint64_t a[CAP];
    if (from_win) {
#pragma unroll
        for (int c = 0; c < CAP; ++c) {
            if (c % 8 == 0) __builtin_amdgcn_sched_barrier(0);
            a[c] = ~0ull;
            if (c < cnt) {
                const int t = list_get(s_list, c, lane);
                const float2 pt = s_xy[t];
                a[c] = make_key(dist2(pt.x, pt.y, qx, qy), s_id[t]);
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < CAP; ++c) {
            if (c % 8 == 0) __builtin_amdgcn_sched_barrier(0);
            a[c] = ~0ull;
            if (c < cnt) {
                const float4 pt = g.P[list_get(s_list, c, lane)];
                a[c] = make_key(dist2(pt.x, pt.y, qx, qy), __float_as_int(pt.z));
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    sort_keys<CAP>(a);
    if constexpr (ROWS) {
        s_gb[lane] = qi;  // the window's row bases are dead: output row of each lane's query
        store_rows_wave<CAP>(a, k, min(WIN_THREADS, M - (int)blockIdx.x * WIN_THREADS), s_gb, s_list, lane, out_idx,
                             idx_i64, out_d2, (int64_t)b * M);
    } else if (active) {
        store_row<CAP>(a, k, out_idx, idx_i64, out_d2, ((int64_t)b * M + qi) * k);
    }
}

// Workgroups of a windowed kernel resident on one CU, queried once per kernel.
static int win_resident_per_cu(const void *fn) {
    constexpr int SLOTS = 8;
    static const void *keys[SLOTS];
    static int vals[SLOTS];
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < SLOTS; ++i)
        if (keys[i] == fn) return vals[i];
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, WIN_THREADS, 0) != hipSuccess || n <= 0) n = 8;
    for (int i = 0; i < SLOTS; ++i)
        if (!keys[i]) {
            keys[i] = fn;
            vals[i] = n;
            break;
        }
    return n;
}

}  // namespace knn
}  // namespace aff

using namespace aff;

namespace {
// Bytes of the grid part of the workspace; the tile-sorted queries follow.
size_t knn_grid_bytes(int B, int N) {
    const grid::Segs s = grid::make_segs(1, &N);
    return grid::ws_layout(B, s).total;
}
}  // namespace

extern "C" size_t aff_knn_workspace_bytes(int B, int M, int N, int D, int k) {
    (void)k;
    if (B <= 0 || N <= 0 || D != 2) return 0;  // the search in other dimensions needs no workspace
    return knn_grid_bytes(B, N) + grid::align256(sizeof(float4) * (size_t)B * (size_t)(M > 0 ? M : 0));
}

extern "C" aff_status aff_knn(const float *query, int64_t q_sb, int64_t q_sm, const float *ref,
                              int64_t r_sb, int64_t r_sn, int B, int M, int N, int D, int k,
                              void *out_idx, int idx_is_i64, float *out_d2, void *ws,
                              size_t ws_bytes, aff_stream_t stream) {
    AFF_CHECK_ARG(B >= 0 && M >= 0, "aff_knn: B=%d and M=%d must be >= 0", B, M);
    AFF_CHECK_ARG(N >= 1, "aff_knn: N=%d must be >= 1", N);
    AFF_CHECK_ARG(k >= 1 && k <= N, "aff_knn: k=%d exceeds number of reference points N=%d (or k < 1)", k, N);
    if (D < 1 || D > 4) return fail(AFF_ERR_UNSUPPORTED, "aff_knn: D=%d not supported (1 <= D <= 4)", D);
    AFF_CHECK_ARG(q_sb >= 0 && q_sm >= 0 && r_sb >= 0 && r_sn >= 0, "aff_knn: negative stride");
    if (B == 0 || M == 0) return AFF_OK;
    AFF_CHECK_ARG(query && ref && out_idx, "aff_knn: NULL query/ref/out_idx");
    if (D != 2)
        return knn_brute_launch(query, q_sb, q_sm, ref, r_sb, r_sn, B, M, N, D, k, out_idx, idx_is_i64, out_d2,
                                static_cast<hipStream_t>(stream));
    const grid::Segs s = grid::make_segs(1, &N);
    const grid::WsLayout L = grid::ws_layout(B, s);
    const size_t need = aff_knn_workspace_bytes(B, M, N, D, k);
    if (!ws || ws_bytes < need)
        return fail(AFF_ERR_WORKSPACE, "aff_knn: workspace of %zu bytes needed, got %zu", need, ws_bytes);
    AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(ws) & 255) == 0, "aff_knn: workspace must be 256-byte aligned");
    AFF_CHECK_ARG(B <= 65535, "aff_knn: B=%d exceeds 65535", B);

    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool windowed = k <= 64 && N <= knn::MAX_SLOT;
    float4 *qsorted = reinterpret_cast<float4 *>(static_cast<char *>(ws) + L.total);
    // sparser queries (M < N / 2) take the wide window and smaller tiles (32 queries,
    // measured faster at cfg3); as dense as the points, 48 (32 was slower at cfg2)
    const bool wide = 2 * (int64_t)M < (int64_t)N;
    const grid::QueryBin qb{query, q_sb, q_sm, M, windowed ? qsorted : nullptr, wide ? 32 : 48};
    aff_status r = grid::launch_build(ref, r_sb, r_sn, B, s, ws, st, qb);
    if (r != AFF_OK) return r;
    dim3 block(knn::QUERY_THREADS);
    dim3 gridd((M + knn::QUERY_THREADS - 1) / knn::QUERY_THREADS, B);
    if (windowed) {
        // sparser queries spread a wave's 64 queries over more points: take the wider window
        using WinFn = void (*)(const float4 *, const grid::Segs, const void *, grid::WsLayout, int, int, void *, int,
                               float *);
        auto pick = [&](bool rows) -> WinFn {
            if (k <= 12)
                return wide ? (rows ? knn::knn_win_kernel<16, knn::WMAX_WIDE, knn::WCMAX_WIDE, true>
                                    : knn::knn_win_kernel<16, knn::WMAX_WIDE, knn::WCMAX_WIDE, false>)
                            : (rows ? knn::knn_win_kernel<16, knn::WMAX, knn::WCMAX, true>
                                    : knn::knn_win_kernel<16, knn::WMAX, knn::WCMAX, false>);
            if (k <= 24)
                return wide ? (rows ? knn::knn_win_kernel<32, knn::WMAX_WIDE, knn::WCMAX_WIDE, true>
                                    : knn::knn_win_kernel<32, knn::WMAX_WIDE, knn::WCMAX_WIDE, false>)
                            : (rows ? knn::knn_win_kernel<32, knn::WMAX, knn::WCMAX, true>
                                    : knn::knn_win_kernel<32, knn::WMAX, knn::WCMAX, false>);
            return wide ? (rows ? knn::knn_win_kernel<64, knn::WMAX_WIDE, knn::WCMAX_WIDE, true>
                                : knn::knn_win_kernel<64, knn::WMAX_WIDE, knn::WCMAX_WIDE, false>)
                        : (rows ? knn::knn_win_kernel<64, knn::WMAX, knn::WCMAX, true>
                                : knn::knn_win_kernel<64, knn::WMAX, knn::WCMAX, false>);
        };
        // More waves than fit at once: the launch is throughput bound; whole-row stores
        // (through LDS) cost the memory path far less than one word per row per store,
        // and the starting radius is refined from the window's cell counts.  One
        // resident generation: the direct stores and unrefined start end each wave sooner.
        const WinFn direct = pick(false);
        const int64_t waves = (int64_t)gridd.x * gridd.y;
        const bool rows =
            waves > (int64_t)knn::win_resident_per_cu(reinterpret_cast<const void *>(direct)) * device_cu_count();
        hipLaunchKernelGGL(rows ? pick(true) : direct, gridd, block, 0, st, qsorted, s, ws, L, M, k, out_idx,
                           idx_is_i64, out_d2);
    } else if (k <= 64) {
        hipLaunchKernelGGL(knn::knn_query_kernel<64>, gridd, block, 0, st, query, q_sb, q_sm, s, ws, L, M, k, out_idx,
                           idx_is_i64, out_d2);
    } else {
        hipLaunchKernelGGL(knn::knn_query_kernel<16>, gridd, block, 0, st, query, q_sb, q_sm, s, ws, L, M, k, out_idx,
                           idx_is_i64, out_d2);
    }
    return check_launch("aff_knn/query");
}

// ------------------------------------------------------------------------
// aff_knn_noalloc: aff_knn with its workspace in a static device array, for
// callers that cannot allocate device memory (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc).
//
// `scratch` is a file-scope device array: in host code its name is only a
// host-side stand-in, never a device address.  The device address is taken
// once per device with hipGetSymbolAddress (with that device current, on the
// entry point's first call there) and kept per device; only that address is
// ever handed to kernels.  Every call on one GPU shares that GPU's array: the
// grid build writes every workspace byte the query kernels read, so nothing
// has to start at zero, but calls that overlap on one GPU (concurrent streams
// or host threads) race on it.
// ------------------------------------------------------------------------
namespace {

static __device__ __align__(256) unsigned char scratch[AFF_KNN_NOALLOC_SCRATCH_BYTES];

constexpr int SCRATCH_MAXDEV = 64;
std::once_flag g_scratch_once[SCRATCH_MAXDEV];
void *g_scratch_ptr[SCRATCH_MAXDEV];
hipError_t g_scratch_err[SCRATCH_MAXDEV];

// The current device's address of `scratch`.
aff_status scratch_address(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_MAXDEV)
        return fail(AFF_ERR_LAUNCH, "aff_knn_noalloc: no usable current device (%d)", dev);
    std::call_once(g_scratch_once[dev], [dev] {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_err[dev] = e;
        g_scratch_ptr[dev] = e == hipSuccess ? p : nullptr;
    });
    if (g_scratch_err[dev] != hipSuccess || g_scratch_ptr[dev] == nullptr)
        return fail(AFF_ERR_LAUNCH, "aff_knn_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                    hipGetErrorString(g_scratch_err[dev]));
    *out = g_scratch_ptr[dev];
    return AFF_OK;
}

}  // namespace

extern "C" aff_status aff_knn_noalloc(const float *query, int64_t q_sb, int64_t q_sm, const float *ref,
                                      int64_t r_sb, int64_t r_sn, int B, int M, int N, int D, int k,
                                      void *out_idx, int idx_is_i64, float *out_d2, aff_stream_t stream) {
    // the argument checks of aff_knn, before the device is touched
    AFF_CHECK_ARG(B >= 0 && M >= 0, "aff_knn_noalloc: B=%d and M=%d must be >= 0", B, M);
    AFF_CHECK_ARG(N >= 1, "aff_knn_noalloc: N=%d must be >= 1", N);
    AFF_CHECK_ARG(k >= 1 && k <= N, "aff_knn_noalloc: k=%d exceeds number of reference points N=%d (or k < 1)", k, N);
    if (D < 1 || D > 4) return fail(AFF_ERR_UNSUPPORTED, "aff_knn_noalloc: D=%d not supported (1 <= D <= 4)", D);
    AFF_CHECK_ARG(q_sb >= 0 && q_sm >= 0 && r_sb >= 0 && r_sn >= 0, "aff_knn_noalloc: negative stride");
    if (B == 0 || M == 0) return AFF_OK;
    AFF_CHECK_ARG(query && ref && out_idx, "aff_knn_noalloc: NULL query/ref/out_idx");
    const size_t need = aff_knn_workspace_bytes(B, M, N, D, k);
    if (need > (size_t)AFF_KNN_NOALLOC_SCRATCH_BYTES)
        return fail(AFF_ERR_WORKSPACE, "aff_knn_noalloc: needs %zu bytes of scratch, the static scratch holds %zu",
                    need, (size_t)AFF_KNN_NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    const aff_status st = scratch_address(&ws);
    if (st != AFF_OK) return st;
    return aff_knn(query, q_sb, q_sm, ref, r_sb, r_sn, B, M, N, D, k, out_idx, idx_is_i64, out_d2, ws,
                   (size_t)AFF_KNN_NOALLOC_SCRATCH_BYTES, stream);
}
