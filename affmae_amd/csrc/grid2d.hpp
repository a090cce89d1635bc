// Uniform-grid exact K-nearest-neighbour machinery shared by the KNN and the
// deformable-attention kernels.
//
// A "segment" is one point set searched on its own: one image for aff_knn,
// one (image, level) pair for deformable attention.  Each segment is
// counting-sorted into ~N/2 cells by grid_build_kernel (knn.hip); queries
// then visit only the cells that can hold points within a radius U.
//
// Order: keys (float bits of d2 << 32 | index) ascending, i.e. by distance
// and, on equal distance, by lower index - the order of the reference's
// streaming kernels (src/layers/kernels/knn.py:313-330, strict '<' insertion
// in index order).  d2 = fl(fl(dx*dx) + fl(dy*dy)) with no contraction.
#pragma once

#include "common.hpp"

#include <math.h>

namespace aff {
namespace grid {

constexpr int MAX_SEGS = 8;        // segments per batch item (levels)
constexpr int BUILD_THREADS = 1024;
constexpr int MAX_CELLS = 16384;   // LDS histogram of the build kernel: 64 KB
constexpr int PTS_PER_CELL = 2;
constexpr int MAX_REFINE = 64;

struct GridParams {
    float x0, y0, h, inv_h;
    int gx, gy, ncell, pad;
};

// Segment table of one batch item; every batch item has the same layout.
struct Segs {
    int L;                       // segments per batch item
    int start[MAX_SEGS + 1];     // point rows of segment l: [start[l], start[l+1])
    int cell_off[MAX_SEGS + 1];  // int offset of segment l's cell array (cmax[l] + 1 entries)
    int cmax[MAX_SEGS];          // cells of segment l
    int64_t cells_per_b;         // ints of cell arrays per batch item
    int npts_b;                  // points per batch item (= start[L])
};

inline int target_cells(int n) {
    int c = n / PTS_PER_CELL;
    if (c < 1) c = 1;
    if (c > MAX_CELLS) c = MAX_CELLS;
    return c;
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Segment table for level sizes n[0..L-1] (host side).
inline Segs make_segs(int L, const int *n) {
    Segs s{};
    s.L = L;
    int off = 0, coff = 0;
    for (int l = 0; l < L; ++l) {
        s.start[l] = off;
        s.cell_off[l] = coff;
        s.cmax[l] = target_cells(n[l]);
        off += n[l];
        coff += s.cmax[l] + 1;
    }
    s.start[L] = off;
    s.cell_off[L] = coff;
    s.cells_per_b = coff;
    s.npts_b = off;
    return s;
}

struct WsLayout {
    size_t params, cells, pts, total;
};

inline WsLayout ws_layout(int B, const Segs &s) {
    WsLayout w;
    size_t off = 0;
    w.params = off;
    off = align256(off + sizeof(GridParams) * (size_t)B * s.L);
    w.cells = off;
    off = align256(off + sizeof(int) * (size_t)B * (size_t)s.cells_per_b);
    w.pts = off;
    off = align256(off + sizeof(float4) * (size_t)B * (size_t)s.npts_b);
    w.total = off;
    return w;
}

// Queries per cell tile of the KNN query sort (see QueryBin), and points per
// build thread kept in registers.
constexpr int TILE_QUERIES = 48;
constexpr int PPT = 8;

// Optional query sort done by the build of a single-segment grid: query
// (b, i) at q[b * q_sb + i * q_sm + {0, 1}], i < M, is written to
// out[b * M + slot] = (x, y, i bits, 0), ordered by the cell tile of the
// grid it falls in.  out == nullptr skips the sort.
struct QueryBin {
    const float *q;
    int64_t q_sb, q_sm;
    int M;
    float4 *out;
    int tile_queries;  // queries per tile; TILE_QUERIES when 0
};

// Optional: ints the build sets to zero before anything that runs after it on
// the stream (allocation counters of later passes).
struct ZeroSpan {
    int *p;
    int n;
};

// Builds the grids of all B * s.L segments (defined in knn.hip).
// src: point (b, row) at src[b * sb + row * sn + {0, 1}], rows as in s.start.
aff_status launch_build(const float *src, int64_t sb, int64_t sn, int B, const Segs &s, void *ws,
                        hipStream_t stream);
aff_status launch_build(const float *src, int64_t sb, int64_t sn, int B, const Segs &s, void *ws,
                        hipStream_t stream, const QueryBin &qb);
aff_status launch_build(const float *src, int64_t sb, int64_t sn, int B, const Segs &s, void *ws,
                        hipStream_t stream, const ZeroSpan &z);

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
// therefore the tie order) is the one a plain fp32 CPU evaluation gives.  The
// empty asm statement hides the products from the optimiser, so neither can be
// fused into the add, whatever contraction mode the including file uses.
__device__ __forceinline__ float dist2(float ax, float ay, float bx, float by) {
    const float dx = ax - bx, dy = ay - by;
    float px = dx * dx, py = dy * dy;
    asm volatile("" : "+v"(px), "+v"(py));
    return px + py;
}

__device__ __forceinline__ uint64_t make_key(float d2, int idx) {
    return (uint64_t(__float_as_uint(d2)) << 32) | uint32_t(idx);
}
__device__ __forceinline__ int key_index(uint64_t k) { return int(uint32_t(k)); }
__device__ __forceinline__ float key_d2(uint64_t k) { return __uint_as_float(uint32_t(k >> 32)); }

// View of one built segment.
struct SegView {
    GridParams p;
    const int *cs;     // cell offsets (ncell + 1 used)
    const float4 *P;   // points in cell order: (x, y, index bits, 0)
    int n;             // points in the segment
};

__device__ __forceinline__ SegView seg_view(const void *ws, const WsLayout &L, const Segs &s, int b, int l) {
    const char *w = static_cast<const char *>(ws);
    SegView v;
    v.p = reinterpret_cast<const GridParams *>(w + L.params)[b * s.L + l];
    v.cs = reinterpret_cast<const int *>(w + L.cells) + (int64_t)b * s.cells_per_b + s.cell_off[l];
    v.P = reinterpret_cast<const float4 *>(w + L.pts) + (int64_t)b * s.npts_b + s.start[l];
    v.n = s.start[l + 1] - s.start[l];
    return v;
}

// Calls f(d2, index) for every point whose computed d2 can be <= U (a
// superset: whole cells whose row band and per-row chord meet a slightly
// enlarged disk).
template <typename F>
__device__ __forceinline__ void visit_disk(const SegView &g, float qx, float qy, float U, float slack, F &&f) {
    const GridParams &p = g.p;
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
        const int beg = g.cs[cy * p.gx + cx0], end = g.cs[cy * p.gx + cx1 + 1];
        for (int t = beg; t < end; ++t) {
            const float4 pt = g.P[t];
            f(dist2(pt.x, pt.y, qx, qy), __float_as_int(pt.z));
        }
    }
}

// Ascending sort in registers: Batcher's odd-even merge sort network (543
// compare-exchanges for 64 keys, against 672 for a bitonic network).  All
// loop bounds are compile-time constants, so every index is a register.
// Scheduling barriers every 16 compare-exchanges keep the compiler from
// interleaving a whole stage, which would hold old and new copies of every
// key at once.
template <int N>
__device__ __forceinline__ void sort_keys(uint64_t (&a)[N]) {
    int n = 0;
#pragma unroll
    for (int p = 1; p < N; p <<= 1)
#pragma unroll
        for (int k = p; k >= 1; k >>= 1)
#pragma unroll
            for (int j = k % p; j + k < N; j += 2 * k)
#pragma unroll
                for (int i = 0; i < k && i < N - j - k; ++i)
                    if ((i + j) / (2 * p) == (i + j + k) / (2 * p)) {
                        const uint64_t x = a[i + j], y = a[i + j + k];
                        const bool sw = x > y;
                        a[i + j] = sw ? y : x;
                        a[i + j + k] = sw ? x : y;
                        if (N > 16 && (++n & 15) == 0) __builtin_amdgcn_sched_barrier(0);
                    }
}

__device__ __forceinline__ float query_slack(const GridParams &p, float qx, float qy) {
    const float gw = float(p.gx) * p.h, gh = float(p.gy) * p.h;
    return 1e-5f * (fabsf(p.x0) + fabsf(p.y0) + gw + gh + fabsf(qx) + fabsf(qy)) + 1e-30f;
}

// Initial radius^2: the disk that would hold `target` points at the density
// of the 5x5 cell window around the query, widened by the query's distance
// to the grid.
__device__ __forceinline__ float initial_radius2(const SegView &g, float qx, float qy, float target) {
    const GridParams &p = g.p;
    const int cx = cell_coord(qx, p.x0, p.inv_h, p.gx), cy = cell_coord(qy, p.y0, p.inv_h, p.gy);
    const int ax0 = max(cx - 2, 0), ax1 = min(cx + 2, p.gx - 1);
    const int ay0 = max(cy - 2, 0), ay1 = min(cy + 2, p.gy - 1);
    // the (at most 5) rows' offsets loaded together, then summed
    int lo[5], hi[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const int y = min(ay0 + i, ay1);
        lo[i] = g.cs[y * p.gx + ax0];
        hi[i] = g.cs[y * p.gx + ax1 + 1];
    }
    int cntw = 0;
#pragma unroll
    for (int i = 0; i < 5; ++i)
        if (ay0 + i <= ay1) cntw += hi[i] - lo[i];
    const float h2 = p.h * p.h;
    const float rho = cntw > 0 ? float(cntw) / (float((ax1 - ax0 + 1) * (ay1 - ay0 + 1)) * h2)
                               : float(g.n) / (float(p.ncell) * h2);
    const float gw = float(p.gx) * p.h, gh = float(p.gy) * p.h;
    const float ex = fmaxf(0.f, fmaxf(p.x0 - qx, qx - (p.x0 + gw)));
    const float ey = fmaxf(0.f, fmaxf(p.y0 - qy, qy - (p.y0 + gh)));
    float rad = sqrtf(target / (3.14159265f * rho));
    // Near the grid's edges part of the disk holds no points: widen the
    // radius by the inverse of the covered fraction of the disk's bounding
    // square (twice, as the fraction shrinks with the new radius).
    if (ex == 0.f && ey == 0.f) {
        const float r0 = rad;
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const float fx = (fminf(qx + rad, p.x0 + gw) - fmaxf(qx - rad, p.x0)) / (2.f * rad);
            const float fy = (fminf(qy + rad, p.y0 + gh) - fmaxf(qy - rad, p.y0)) / (2.f * rad);
            const float f = fmaxf(fx * fy, 0.0625f);
            rad = r0 * sqrtf(1.f / f);
        }
    }
    rad += sqrtf(ex * ex + ey * ey);
    float U = fmaxf(rad * rad, 1e-30f);
    return U < INFINITY ? U : INFINITY;
}

// Exact k nearest neighbours of (qx, qy) in segment g, 1 <= k <= CAP and
// k <= g.n.  On return a[0..k-1] hold the k smallest keys in ascending order
// (a[k..CAP-1] = ~0).  `col` is this lane's LDS column of CAP keys with
// element stride `stride`.
template <int CAP>
__device__ __forceinline__ void knn_select(const SegView &g, float qx, float qy, int k, uint64_t *col, int stride,
                                           uint64_t (&a)[CAP]) {
    const float slack = query_slack(g.p, qx, qy);
    const float target = 0.5f * float(k + CAP);
    float U = initial_radius2(g, qx, qy, target);
    float lo = -1.f, hi = INFINITY;
    int cnt = -1;
    bool ok = false;
    for (int it = 0; it < MAX_REFINE; ++it) {
        int c = 0;
        const float Uc = U;
        visit_disk(g, qx, qy, Uc, slack, [&](float d2, int idx) {
            if (d2 <= Uc) {
                if (c < CAP) col[c * stride] = make_key(d2, idx);
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
    if (ok) {
#pragma unroll
        for (int s = 0; s < CAP; ++s) a[s] = (s < cnt) ? col[s * stride] : ~0ull;
        sort_keys<CAP>(a);
#pragma unroll
        for (int s = 0; s < CAP; ++s)
            if (s >= k) a[s] = ~0ull;
        return;
    }
    // Exact fallback (ties at one distance): k passes, each taking the
    // smallest key above the previous one, staged through the LDS column.
    const float Uf = (hi < INFINITY) ? hi : INFINITY;
    uint64_t last = 0;
    for (int j = 0; j < k; ++j) {
        uint64_t best = ~0ull;
        const bool first = (j == 0);
        visit_disk(g, qx, qy, Uf, slack, [&](float d2, int idx) {
            if (d2 <= Uf) {
                const uint64_t key = make_key(d2, idx);
                if ((first || key > last) && key < best) best = key;
            }
        });
        col[j * stride] = best;
        last = best;
    }
#pragma unroll
    for (int s = 0; s < CAP; ++s) a[s] = (s < k) ? col[s * stride] : ~0ull;
}

}  // namespace grid
}  // namespace aff
