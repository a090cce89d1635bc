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
// Two launches after the coarse grid build (grid2d.hpp): cand_build_kernel
// writes, for every cell of a finer grid over each level, the list of points
// that can be among the K nearest of any location in the cell (nearest first,
// with lower bounds on the distances); deform_cand_kernel then gives each
// sample one lane that scans its cell's list (exact (d2, row) keys) until the
// bounds pass its K-th distance, stages (row, attn * w) pairs in the wave's
// LDS slice, and gathers the value rows (8 channels per lane, 16-byte loads)
// in fp32.  The neighbour indices never go to HBM unless the caller asks for
// them.
//
// aff_deform_sample_fwd: the same weights from given neighbour indices
//   (fused_deformable_attention, fused_deform_attn.py:79-231, 503-571: sqrt(d2) + 1e-6;
//    mssample, mssample.py:17-125, 300-342: sqrt(d2 + 1e-6)); optional gather.
//
// aff_msdetrpc_fwd: out[b,n,:] = sum_m sum_k attn[b,n,m] * w[b,n,m,k] * val[b, idx[b,n,m,k], :]
//   (msdetrpc.py:25-109).
#include "grid2d.hpp"

#include <limits.h>

namespace aff {
namespace deform {

using namespace grid;

constexpr int THREADS = 256;
constexpr int KMAX = 8;    // neighbours per sample
constexpr int NB = 8;      // value rows in flight per lane (given-index kernels)
constexpr int PAIR_GROUP = 8;   // the deformable gather's rows in flight per lane; pair lists pad to a multiple

// Fine-cell candidate lists.  Every (image, level) gets a second, finer grid
// (cells of FINE x FINE per coarse cell, FPAD coarse cells of margin around
// the coarse grid).  The list of a fine cell holds every point that can be
// among the K nearest of ANY location inside the cell: with R = the K-th
// smallest over the points of their largest distance to the cell rectangle,
// each location of the cell has K points within sqrt(R), so its K nearest
// lie within sqrt(R) of it and hence within sqrt(R) of the rectangle.  A
// sample then scans one short contiguous list, exactly.
constexpr int FINE = 2;          // fine cells per coarse cell side
constexpr int FPAD = 2;          // coarse cells of margin around the coarse grid
constexpr int CB = 256;          // fine cells per build tile (one workgroup)
constexpr int MAX_CAND = 128;    // longest list kept; a longer one sends its samples to the coarse grid

struct FineParams {
    float x0, y0, s, inv_s;  // origin and cell side
    int gx, gy;              // 0 x 0: no fine grid (every sample searches the coarse grid)
    float slack;             // absolute rounding allowance of the cell rectangles
    int pad;
};

// A list entry: the point and its row in the image's level concatenation.  A
// list starts with its HEAD points nearest to the cell sorted by that distance
// (the head), so within the head the distance of an entry to the cell bounds
// the distances of every later entry from below.
// Entries are stored four to a block, the rows apart from the points, so that a
// scan step reads a block as three 16-byte loads and the build writes an entry
// with two stores (lists start and end on block boundaries).
struct alignas(16) CandBlock {
    float2 xy[4];
    int row[4];
};
__device__ __forceinline__ void put_cand(CandBlock *blk, int slot, float x, float y, int row) {
    CandBlock &c = blk[slot >> 2];
    c.xy[slot & 3] = make_float2(x, y);
    c.row[slot & 3] = row;
}

// Workspace of aff_deform_fwd: the coarse grids (grid2d.hpp), then the fine
// grids' parameters, their (begin, count) cell tables, one pool allocation
// counter per batch item (zeroed by the grid build) and the candidate pools.
struct DLayout {
    WsLayout g;
    size_t fparams, fcell, counter, pool, total;
    int fc_off[MAX_SEGS + 1];    // fine-cell table offset of each level (int2 entries)
    int fcmax[MAX_SEGS];         // fine cells reserved per level
    int tile_off[MAX_SEGS + 1];  // first build tile of each level
    int64_t fc_per_b, pool_per_b;
    int tt_per_b;
};

inline int pool_per_point(int K) { return 16 + 8 * K; }

inline DLayout d_layout(int B, const Segs &s, int K) {
    DLayout d{};
    d.g = ws_layout(B, s);
    size_t off = d.g.total;
    d.fparams = off;
    off = align256(off + sizeof(FineParams) * (size_t)B * s.L);
    int fc = 0, tt = 0;
    for (int l = 0; l < s.L; ++l) {
        const int cm = s.cmax[l];
        int sq = 1;
        while (sq * sq < cm) ++sq;
        d.fc_off[l] = fc;
        d.fcmax[l] = FINE * FINE * (cm + 4 * FPAD * (sq + 2) + 4 * FPAD * FPAD);
        fc += d.fcmax[l];
        d.tile_off[l] = tt;
        tt += (d.fcmax[l] + CB - 1) / CB;
    }
    d.fc_off[s.L] = fc;
    d.tile_off[s.L] = tt;
    d.fc_per_b = fc;
    d.tt_per_b = tt;
    d.fcell = off;
    off = align256(off + sizeof(int2) * (size_t)B * fc);
    d.counter = off;
    off = align256(off + sizeof(int) * (size_t)B);
    d.pool_per_b = (int64_t)pool_per_point(K) * s.npts_b + 1024;
    d.pool = off;
    off = align256(off + sizeof(CandBlock) * ((size_t)B * (size_t)d.pool_per_b / 4));
    d.total = off;
    return d;
}

__device__ __forceinline__ int64_t load_index(const void *p, int is_i64, int64_t i) {
    return is_i64 ? static_cast<const int64_t *>(p)[i] : int64_t(static_cast<const int32_t *>(p)[i]);
}

// keys[0 .. KT) ascending; insert `key` if it is smaller than keys[KT - 1].
template <int KT>
__device__ __forceinline__ void topk_insert(uint64_t (&keys)[KT], uint64_t key) {
    bool c[KT];
#pragma unroll
    for (int i = 0; i < KT; ++i) c[i] = key < keys[i];
#pragma unroll
    for (int i = KT - 1; i > 0; --i) keys[i] = c[i - 1] ? keys[i - 1] : (c[i] ? key : keys[i]);
    keys[0] = c[0] ? key : keys[0];
}

// Exact K nearest points of (qx, qy) over one level's coarse grid, keys
// (d2, row) ascending in keys[0 .. keff): the disk d2 <= U grows until the
// keff-th key lies inside it.
template <int KT>
__device__ __forceinline__ void topk_global(const SegView &g, float qx, float qy, float U, int keff,
                                            uint64_t (&keys)[KT]) {
    const float slack = query_slack(g.p, qx, qy);
    const GridParams &p = g.p;
    for (;;) {
#pragma unroll
        for (int i = 0; i < KT; ++i) keys[i] = ~0ull;
        const float r = sqrtf(U) * 1.00002f + slack;
        const int cy0 = cell_coord(qy - r, p.y0, p.inv_h, p.gy), cy1 = cell_coord(qy + r, p.y0, p.inv_h, p.gy);
        for (int cy = cy0; cy <= cy1; ++cy) {
            const float rlo = p.y0 + float(cy) * p.h, rhi = rlo + p.h;
            const float dy = fmaxf(0.f, fmaxf(rlo - qy, qy - rhi) - slack);
            const float w2 = r * r - dy * dy;
            if (!(w2 >= 0.f)) continue;
            const float hw = sqrtf(w2) + slack;
            const int cx0 = cell_coord(qx - hw, p.x0, p.inv_h, p.gx), cx1 = cell_coord(qx + hw, p.x0, p.inv_h, p.gx);
            const int beg = g.cs[cy * p.gx + cx0], end = g.cs[cy * p.gx + cx1 + 1];
            for (int t = beg; t < end; t += 4) {  // four loads in flight per step
                float4 pt[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) pt[u] = g.P[min(t + u, end - 1)];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (t + u < end) topk_insert<KT>(keys, make_key(dist2(pt[u].x, pt[u].y, qx, qy), __float_as_int(pt[u].z)));
            }
        }
        const uint64_t kth = keys[keff - 1 < KT ? keff - 1 : KT - 1];
        if ((kth != ~0ull && key_d2(kth) <= U) || !(U < INFINITY)) return;
        U = fmaxf(U * 2.f, kth != ~0ull ? key_d2(kth) : U);
    }
}

// ------------------------------------------------------ candidate lists --
// Fine grid of one level: the coarse grid's box widened by FPAD coarse cells,
// cells of side h / FINE, widened (x 1.0625 steps) until at most fcmax cells.
__device__ __forceinline__ FineParams fine_params(const GridParams &p, int n, int fcmax) {
    FineParams f{};
    const float pad = float(FPAD) * p.h;
    const float wd = float(p.gx) * p.h + 2.f * pad, ht = float(p.gy) * p.h + 2.f * pad;
    f.x0 = p.x0 - pad;
    f.y0 = p.y0 - pad;
    float s = p.h / float(FINE);
    int gx = 0, gy = 0;
    if (n > 0 && s > 0.f && wd < INFINITY && ht < INFINITY && f.x0 > -INFINITY && f.y0 > -INFINITY &&
        wd / s < 1e6f && ht / s < 1e6f) {
        for (int it = 0; it < 256; ++it) {
            gx = int(wd / s) + 1;
            gy = int(ht / s) + 1;
            if ((int64_t)gx * gy <= fcmax) break;
            s *= 1.0625f;
            gx = gy = 0;
        }
    }
    f.s = s;
    f.inv_s = 1.f / s;
    f.gx = gx;
    f.gy = gy;
    f.slack = 1e-5f * (fabsf(f.x0) + fabsf(f.y0) + wd + ht) + 1e-30f;
    return f;
}

struct Rect {
    float x0, y0, x1, y1;
};

// The count and fill passes must agree on every list bit for bit: the
// geometry below is evaluated without contraction in both.
__device__ __forceinline__ Rect fine_rect(const FineParams &f, int c) {
#pragma clang fp contract(off)
    const int cy = c / f.gx, cx = c - cy * f.gx;
    Rect r;
    r.x0 = f.x0 + float(cx) * f.s - f.slack;
    r.x1 = f.x0 + float(cx + 1) * f.s + f.slack;
    r.y0 = f.y0 + float(cy) * f.s - f.slack;
    r.y1 = f.y0 + float(cy + 1) * f.s + f.slack;
    return r;
}

// R of one fine cell: the keff-th smallest largest-distance^2 from a point to
// the rectangle, over the points of the coarse rings around the rectangle's
// centre (at least the 3 x 3 block; any keff points give a valid bound, the
// nearest ones a tight one).
template <int KT>
__device__ __forceinline__ float cell_bound(const SegView &g, const Rect &rc, int keff) {
#pragma clang fp contract(off)
    const GridParams &p = g.p;
    float top[KT];
#pragma unroll
    for (int i = 0; i < KT; ++i) top[i] = INFINITY;
    int found = 0;
    const int ccx = cell_coord(0.5f * (rc.x0 + rc.x1), p.x0, p.inv_h, p.gx);
    const int ccy = cell_coord(0.5f * (rc.y0 + rc.y1), p.y0, p.inv_h, p.gy);
    auto visit = [&](int cy, int cx0, int cx1) {
        const int beg = g.cs[cy * p.gx + cx0], end = g.cs[cy * p.gx + cx1 + 1];
        for (int t = beg; t < end; t += 4) {  // four loads in flight per step
            float4 pt[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) pt[u] = g.P[min(t + u, end - 1)];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float mx = fmaxf(fabsf(pt[u].x - rc.x0), fabsf(pt[u].x - rc.x1));
                const float my = fmaxf(fabsf(pt[u].y - rc.y0), fabsf(pt[u].y - rc.y1));
                float v = t + u < end ? mx * mx + my * my : INFINITY;
#pragma unroll
                for (int i = 0; i < KT; ++i) {
                    const float lo = fminf(top[i], v);
                    v = fmaxf(top[i], v);
                    top[i] = lo;
                }
            }
        }
        found += end - beg;
    };
    for (int rad = 0;; ++rad) {
        const int ax0 = ccx - rad, ax1 = ccx + rad, ay0 = ccy - rad, ay1 = ccy + rad;
        const int ylo = max(ay0, 0), yhi = min(ay1, p.gy - 1);
        for (int cy = ylo; cy <= yhi; ++cy) {
            if (cy == ay0 || cy == ay1) {
                visit(cy, max(ax0, 0), min(ax1, p.gx - 1));
            } else {
                if (ax0 >= 0) visit(cy, ax0, ax0);
                if (ax1 < p.gx) visit(cy, ax1, ax1);
            }
        }
        const bool full = ax0 <= 0 && ay0 <= 0 && ax1 >= p.gx - 1 && ay1 >= p.gy - 1;
        if ((found >= keff && rad >= 1) || full) break;
    }
    float R = top[0];
#pragma unroll
    for (int i = 1; i < KT; ++i)
        if (i < keff) R = top[i];
    return R * 1.0001f + 1e-30f;
}

// Calls f(point, distance^2 to the rectangle) for every point of the level
// whose distance^2 to the rectangle is at most R, in the coarse grid's cell
// order.
template <typename F>
__device__ __forceinline__ void visit_cands(const SegView &g, const Rect &rc, float R, F &&f) {
#pragma clang fp contract(off)
    const GridParams &p = g.p;
    const float rr = sqrtf(R) * 1.00002f + query_slack(p, rc.x0, rc.y0);
    const int cy0 = cell_coord(rc.y0 - rr, p.y0, p.inv_h, p.gy), cy1 = cell_coord(rc.y1 + rr, p.y0, p.inv_h, p.gy);
    const int cx0 = cell_coord(rc.x0 - rr, p.x0, p.inv_h, p.gx), cx1 = cell_coord(rc.x1 + rr, p.x0, p.inv_h, p.gx);
    for (int cy = cy0; cy <= cy1; ++cy) {
        const int beg = g.cs[cy * p.gx + cx0], end = g.cs[cy * p.gx + cx1 + 1];
        for (int t = beg; t < end; t += 4) {  // four loads in flight per step
            float4 pt[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) pt[u] = g.P[min(t + u, end - 1)];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float dx = fmaxf(0.f, fmaxf(rc.x0 - pt[u].x, pt[u].x - rc.x1));
                const float dy = fmaxf(0.f, fmaxf(rc.y0 - pt[u].y, pt[u].y - rc.y1));
                const float md = dx * dx + dy * dy;
                if (t + u < end && md <= R) f(pt[u], md);
            }
        }
    }
}

struct BArgs {
    Segs segs;
    WsLayout wl;
    const void *ws;
    FineParams *fp;  // [B * L]
    int2 *fcell;     // [B][fc_per_b]: (begin, count) of each fine cell's list
    int *counter;    // [B]: pool entries handed out per batch item
    CandBlock *pool;  // [B][pool_per_b / 4]
    int fc_off[MAX_SEGS + 1], fcmax[MAX_SEGS], tile_off[MAX_SEGS + 1];
    int64_t fc_per_b, pool_per_b;
    int tt_per_b, K;
};

// Exclusive prefix of v over the 256 threads; *total gets the sum.
__device__ __forceinline__ int block_scan(int v, int *s_w, int *total) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) s_w[wid] = incl;
    __syncthreads();
    int off = 0;
    for (int i = 0; i < wid; ++i) off += s_w[i];
    *total = s_w[0] + s_w[1] + s_w[2] + s_w[3];
    __syncthreads();
    return off + incl - v;
}

__device__ __forceinline__ void tile_of(const BArgs &ba, int &b, int &l, int &t, int &gt) {
    b = blockIdx.x / ba.tt_per_b;
    gt = blockIdx.x - b * ba.tt_per_b;
    l = 0;
    while (l + 1 < ba.segs.L && gt >= ba.tile_off[l + 1]) ++l;
    t = gt - ba.tile_off[l];
}

// One lane per fine cell.  Pass 1 over the candidates counts them and keeps
// their HEAD smallest distances to the cell; the tile's lists then get pool
// space from the image's counter (one atomic per tile: the layout depends on
// the order tiles arrive in, the lists do not).  Pass 2 writes each of those
// HEAD nearest points at its rank among them (the sorted head) and the rest
// after them in visit order.  Each list is padded to a multiple of 4 entries
// with points at infinity; its cell entry holds (begin, padded length | head
// length << 16).  Lists longer than MAX_CAND, or beyond the pool, get count
// -1: their samples search the coarse grid.
constexpr int HEAD = 12;  // sorted head length: 16 and 8 both timed slower at cfg4

template <int KT>
__global__ __launch_bounds__(CB) void cand_build_kernel(const BArgs ba) {
    __shared__ int s_w[4];
    __shared__ int s_base;
    int b, l, t, gt;
    tile_of(ba, b, l, t, gt);
    const SegView g = seg_view(ba.ws, ba.wl, ba.segs, b, l);
    const FineParams f = fine_params(g.p, g.n, ba.fcmax[l]);
    if (t == 0 && threadIdx.x == 0) ba.fp[b * ba.segs.L + l] = f;
    const int ncf = f.gx * f.gy;
    if (t * CB >= ncf) return;  // the whole tile lies beyond the grid
    const int c = t * CB + threadIdx.x;
    const bool valid = c < ncf && g.n > 0;
    Rect rc{};
    float R = 0.f;
    int cnt = 0;
    float top[HEAD];
#pragma unroll
    for (int i = 0; i < HEAD; ++i) top[i] = INFINITY;
    if (valid) {
        rc = fine_rect(f, c);
        R = cell_bound<KT>(g, rc, min(ba.K, g.n));
        visit_cands(g, rc, R, [&](const float4 &, float md) {
            ++cnt;
            float v = md;
#pragma unroll
            for (int i = 0; i < HEAD; ++i) {
                const float lo = fminf(top[i], v);
                v = fmaxf(top[i], v);
                top[i] = lo;
            }
        });
    }
    if (cnt > MAX_CAND) cnt = -1;
    const int cnt4 = (max(cnt, 0) + 3) & ~3;  // lists padded to whole 4-entry steps
    int tot;
    const int pre = block_scan(cnt4, s_w, &tot);
    if (threadIdx.x == 0) s_base = tot > 0 ? atomicAdd(ba.counter + b, tot) : 0;
    __syncthreads();
    if (c >= ncf) return;
    const int64_t begin = (int64_t)s_base + pre;
    if (cnt > 0 && begin + cnt4 > ba.pool_per_b) cnt = -1;
    const int m = min(max(cnt, 0), HEAD);
    ba.fcell[b * ba.fc_per_b + ba.fc_off[l] + c] = make_int2(cnt > 0 ? int(begin) : 0, cnt > 0 ? cnt4 | (m << 16) : cnt);
    if (cnt <= 0) return;
    CandBlock *out = ba.pool + (b * ba.pool_per_b + begin) / 4;  // both multiples of 4
    // padding: points at infinity (their keys lose to every real point)
    for (int i = cnt; i < cnt4; ++i) put_cand(out, i, INFINITY, INFINITY, -1);
    float tb = top[0];
#pragma unroll
    for (int i = 1; i < HEAD; ++i)
        if (i < m) tb = top[i];
    uint32_t used = 0;
    int tail = m;
    visit_cands(g, rc, R, [&](const float4 &pt, float md) {
        int slot = HEAD;
        if (md <= tb) {
            int rank = 0;
#pragma unroll
            for (int i = 0; i < HEAD; ++i) rank += top[i] < md ? 1 : 0;
            while (rank < m && ((used >> rank) & 1u)) ++rank;  // equal distances take the next free slot
            slot = rank;
        }
        if (slot < m) used |= 1u << slot;
        else slot = tail++;
        if (slot < cnt) put_cand(out, slot, pt.x, pt.y, __float_as_int(pt.z));
    });
}

// --------------------------------------------------------- main kernel --
struct CArgs {
    aff_deform_args a;
    Segs segs;
    WsLayout wl;
    const void *ws;
    const FineParams *fp;
    const int2 *fcell;
    const CandBlock *pool;
    int fc_off[MAX_SEGS + 1];
    int64_t fc_per_b, pool_per_b;
    int pl_log2;  // lanes per row = 2^pl_log2 >= P
    int osz, asz;  // bytes per offset / attention element
};

// Raw bits of a sample's offset pair and attention weight, read with
// dtype-independent instructions: a 16-bit pair is one dword (read twice), an
// fp32 pair two; a 16-bit weight one half-word (read twice), an fp32 weight
// two.  Nothing is read outside the element.
__device__ __forceinline__ void load_sample_raw(const char *op, const char *ap, int osz, int asz, uint32_t &o0,
                                                uint32_t &o1, uint32_t &at) {
    o0 = *reinterpret_cast<const uint32_t *>(op);
    o1 = *reinterpret_cast<const uint32_t *>(op + (osz == 4 ? 4 : 0));
    const uint32_t lo = *reinterpret_cast<const uint16_t *>(ap);
    const uint32_t hi = *reinterpret_cast<const uint16_t *>(ap + (asz == 4 ? 2 : 0));
    at = lo | (hi << 16);
}

__device__ __forceinline__ float raw_to_float(uint32_t v, int dtype) {
    if (dtype == AFF_F32) return __uint_as_float(v);
    if (dtype == AFF_BF16) return __uint_as_float(v << 16);
    return float(__builtin_bit_cast(_Float16, uint16_t(v)));
}

// One wave = RW = 64 / PL consecutive (b, q, h) rows.  Search: lane (r, p)
// takes sample (l, p) of row r for every level l.  Every level's sample
// (offset, weight, fine-cell parameters) is read first, then every level's
// cell entry, so those reads overlap; then each level's list is scanned
// (four entries per step, the next four in flight, until the entries' bound
// passes the K-th distance) or, outside the fine grid,
// the coarse grid searched, and (value offset, attn * w) of the K neighbours
// staged in the wave's LDS slice.  Gather: lane (r, chunk) sums the row's
// L * P * K value rows over 8 channels (16-byte loads) in fp32.  Waves share
// nothing; the workgroup only batches them.
template <typename T, int KT, int LMAX>
__global__ __launch_bounds__(THREADS) void deform_cand_kernel(const CArgs ka) {
    using IO = ElemIO<T>;
    extern __shared__ int2 s_pair[];
    const aff_deform_args &a = ka.a;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nwv = blockDim.x >> 6;
    const int PL = 1 << ka.pl_log2, RW = 64 >> ka.pl_log2;
    const int L = a.L, S = L * a.P, K = a.K, SK = S * K;
    const int SKP = (SK + PAIR_GROUP - 1) / PAIR_GROUP * PAIR_GROUP;  // pairs per row, padded
    int2 *pr = s_pair + wv * RW * SKP;
    const int64_t total = (int64_t)a.B * a.Nq * a.H;
    const int64_t row0 = ((int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * nwv + wv) * RW;
    const float pw = *a.power;
    const int ipow = (pw == 0.f || pw == 1.f || pw == 2.f || pw == 3.f || pw == 4.f) ? int(pw) : -1;

    {
        const int r = lane >> ka.pl_log2, p = lane & (PL - 1);
        const int64_t row = row0 + r;
        const bool act = row < total && p < a.P;
        const uint32_t rw = act ? uint32_t(row) : 0u;  // the host keeps B * Nq * H below 2^31
        const int pc = act ? p : 0;
        const int h = int(rw % uint32_t(a.H));
        const uint32_t bq = rw / uint32_t(a.H);
        const int q = int(bq % uint32_t(a.Nq)), b = int(bq / uint32_t(a.Nq));
        const float qx = a.query_pos[(int64_t)b * a.qp_sb + (int64_t)q * a.qp_sn];
        const float qy = a.query_pos[(int64_t)b * a.qp_sb + (int64_t)q * a.qp_sn + 1];
        const char *ob = static_cast<const char *>(a.offsets) +
                         ((int64_t)b * a.off_sb + (int64_t)q * a.off_sn + (int64_t)h * a.off_sh) * ka.osz;
        const char *abase = static_cast<const char *>(a.attn) +
                            ((int64_t)b * a.at_sb + (int64_t)q * a.at_sn + (int64_t)h * a.at_sh) * ka.asz;
        const int2 *fc_b = ka.fcell + b * ka.fc_per_b;
        const int vrow = h * int(a.v_sh);  // value offset of head h (elements; the host keeps it below 2^31)
        if (act && p == 0)  // the row's padding pairs: a valid row with weight 0
            for (int j = SK; j < SKP; ++j) pr[r * SKP + j] = make_int2(vrow, 0);
        // The fine-grid parameters come through the scalar cache when the wave's
        // rows all lie in one image (always, unless an image has fewer rows than
        // a wave), through vector loads otherwise.
        const int b0 = __builtin_amdgcn_readfirstlane(b);
        const bool uni = __all(b == b0);

        // ---- every level's sample (levels >= L repeat level L - 1)
        uint32_t o0[LMAX], o1[LMAX], at[LMAX];
#pragma unroll
        for (int l = 0; l < LMAX; ++l) {
            const int lc = min(l, L - 1);
            const int s = lc * a.P + pc;
            load_sample_raw(ob + s * 2 * ka.osz, abase + s * ka.asz, ka.osz, ka.asz, o0[l], o1[l], at[l]);
        }
        // ---- sample locations and every level's cell entry
        float sxl[LMAX], syl[LMAX];
        int2 ce[LMAX];
        bool inside[LMAX];
        auto locate = [&](const FineParams *fpb) {
#pragma unroll
            for (int l = 0; l < LMAX; ++l) {
#pragma clang fp contract(off)
                const int lc = min(l, L - 1);
                const FineParams f = fpb[lc];
                sxl[l] = qx + raw_to_float(o0[l], a.off_dtype);
                syl[l] = qy + raw_to_float(a.off_dtype == AFF_F32 ? o1[l] : o0[l] >> 16, a.off_dtype);
                const float fx = floorf(__fmul_rn(__fsub_rn(sxl[l], f.x0), f.inv_s));
                const float fy = floorf(__fmul_rn(__fsub_rn(syl[l], f.y0), f.inv_s));
                inside[l] = fx >= 0.f && fx < float(f.gx) && fy >= 0.f && fy < float(f.gy);
                const int cell = inside[l] ? int(fy) * f.gx + int(fx) : 0;
                ce[l] = fc_b[ka.fc_off[lc] + cell];
            }
        };
        if (uni) locate(ka.fp + b0 * L);
        else locate(ka.fp + b * L);

        // Levels in turn: level l's values sit at index 0 of the staged arrays,
        // which shift down by one after each level (constant indices keep
        // them in registers with a runtime level loop).
        for (int l = 0; l < L; ++l) {
            const int s = l * a.P + p;
            const int lstart = ka.segs.start[l];
            const int keff = min(K, ka.segs.start[l + 1] - lstart);
            const float sx = sxl[0], sy = syl[0];
            uint64_t keys[KT];
#pragma unroll
            for (int j = 0; j < KT; ++j) keys[j] = ~0ull;
            const int cy_raw = act && keff > 0 ? (inside[0] ? ce[0].y : -1) : 0;
            const int cnt = cy_raw > 0 ? cy_raw & 0xffff : cy_raw, head = cy_raw > 0 ? cy_raw >> 16 : 0;
            if (cnt > 0) {
                // Lists are padded to whole 4-entry blocks (points at infinity); a
                // lane reads one block per step.  Within the sorted head a lane stops
                // once a block's last entry is farther from the cell than its K-th
                // distance: the head is sorted by that distance, computed here exactly
                // as the build computed it (same widened rectangle, no contraction),
                // and the tail's entries are no nearer to the cell than the head's, so
                // it bounds every later entry from below (scaled down a little against
                // the rounding of either distance).  An unfilled K-th key reads as
                // NaN, which never compares less.
                FineParams f;
                if (uni) f = ka.fp[b0 * L + l];
                else f = ka.fp[b * L + l];
                Rect rc;
                {
#pragma clang fp contract(off)
                    const int cx = int(floorf(__fmul_rn(__fsub_rn(sx, f.x0), f.inv_s)));
                    const int cy = int(floorf(__fmul_rn(__fsub_rn(sy, f.y0), f.inv_s)));
                    rc = fine_rect(f, cy * f.gx + cx);
                }
                auto below = [&](const CandBlock &e) {  // the block's last entry
#pragma clang fp contract(off)
                    const float dx = fmaxf(0.f, fmaxf(rc.x0 - e.xy[3].x, e.xy[3].x - rc.x1));
                    const float dy = fmaxf(0.f, fmaxf(rc.y0 - e.xy[3].y, e.xy[3].y - rc.y1));
                    return (dx * dx + dy * dy) * 0.999996f > key_d2(keys[KT - 1]);
                };
                const CandBlock *cp = ka.pool + (b * ka.pool_per_b + ce[0].x) / 4;  // both multiples of 4
                const bool can_stop = keff == KT;
                CandBlock blk = cp[0];
                for (int i = 0;; i += 4) {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        topk_insert<KT>(keys, make_key(dist2(blk.xy[u].x, blk.xy[u].y, sx, sy), blk.row[u]));
                    // entry i + 3 in the head bounds every later entry
                    if (i + 4 >= cnt || (can_stop && i + 4 <= head && below(blk))) break;
                    blk = cp[i / 4 + 1];
                }
            } else if (cnt < 0) {
                const SegView g = seg_view(ka.ws, ka.wl, ka.segs, b, l);
                const float area = float(g.p.gx) * float(g.p.gy) * g.p.h * g.p.h;
                const float rho = float(g.n) / fmaxf(area, 1e-30f);
                const float U0 = keff >= g.n ? INFINITY : fmaxf(float(keff + 4) / (3.14159265f * rho), 1e-30f);
                topk_global<KT>(g, sx, sy, U0, keff, keys);
            }
            // ---- this sample's neighbours: value offsets and weights (none for
            // inactive lanes)
            int nb[KT];
            float wt[KT];
            {
                const float aw = act ? raw_to_float(at[0], a.attn_dtype) : 0.f;
                float wj[KT];
                float wsum = 0.f;
                if (a.mode == AFF_DEFORM_SHEPARD) {
                    const float pp = fmaxf(pw, 1e-6f);
                    float lg[KT], mx = -INFINITY;
#pragma unroll
                    for (int j = 0; j < KT; ++j) {
                        lg[j] = j < keff ? -pp * (__builtin_amdgcn_sqrtf(key_d2(keys[j])) + 1e-6f) : -INFINITY;
                        mx = fmaxf(mx, lg[j]);
                    }
#pragma unroll
                    for (int j = 0; j < KT; ++j) {
                        wj[j] = j < keff ? __expf(lg[j] - mx) : 0.f;
                        wsum += wj[j];
                    }
                    wsum += 1e-8f;
                } else {
                    // d2^power: a product chain for the integer powers 0..4 (exact to a few
                    // ulp), exp2(power * log2(d2)) otherwise
#pragma unroll
                    for (int j = 0; j < KT; ++j) {
                        const float d2 = key_d2(keys[j]);
                        float pv;
                        if (ipow == 0) pv = 1.f;
                        else if (ipow == 1) pv = d2;
                        else if (ipow == 2) pv = d2 * d2;
                        else if (ipow == 3) pv = d2 * d2 * d2;
                        else if (ipow == 4) pv = (d2 * d2) * (d2 * d2);
                        else pv = __builtin_amdgcn_exp2f(pw * __builtin_amdgcn_logf(d2));
                        wj[j] = j < keff ? __builtin_amdgcn_rcpf(pv + 1e-10f) : 0.f;
                        wsum += wj[j];
                    }
                    wsum += 1e-12f;
                }
                const float inv = __builtin_amdgcn_rcpf(wsum);
#pragma unroll
                for (int j = 0; j < KT; ++j) {
                    const bool ok = act && j < keff && j < K;
                    nb[j] = ok ? key_index(keys[j]) * int(a.v_sn) + vrow : -1;
                    wt[j] = ok ? aw * wj[j] * inv : 0.f;
                }
            }
            if (act) {
                int2 *dst = pr + r * SKP + s * K;
#pragma unroll
                for (int j = 0; j < KT; ++j)
                    if (j < K) dst[j] = make_int2(nb[j] >= 0 ? nb[j] : vrow, __float_as_int(wt[j]));
            }
            if (act && (a.knn_idx || a.knn_d2)) {
                const int64_t kb = (row * S + s) * K;  // [B, Nq, H, L, P, K]
#pragma unroll
                for (int j = 0; j < KT; ++j) {
                    if (j < K) {
                        const bool ok = j < keff;
                        if (a.knn_idx) a.knn_idx[kb + j] = ok ? key_index(keys[j]) - lstart : -1;
                        if (a.knn_d2) a.knn_d2[kb + j] = ok ? key_d2(keys[j]) : INFINITY;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i + 1 < LMAX; ++i) {
                sxl[i] = sxl[i + 1];
                syl[i] = syl[i + 1];
                ce[i] = ce[i + 1];
                inside[i] = inside[i + 1];
                at[i] = at[i + 1];
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- gather: each row's SKP pairs (value offset of (row, head) in elements,
    // weight; the padding has weight 0); GB rows in flight per lane, pairs read
    // two per LDS access
    constexpr int GB = PAIR_GROUP;
    const int CG = a.C / 8;
    for (int it = lane; it < RW * CG; it += 64) {
        const int rr = it / CG, cc = it - rr * CG;
        const int64_t row = row0 + rr;
        if (row >= total) break;  // rows ascend with it
        const uint32_t rw = uint32_t(row);
        const int h = int(rw % uint32_t(a.H));
        const uint32_t bq = rw / uint32_t(a.H);
        const int q = int(bq % uint32_t(a.Nq)), b = int(bq / uint32_t(a.Nq));
        const T *V = static_cast<const T *>(a.values) + (int64_t)b * a.v_sb + cc * 8;
        T *O = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)q * a.o_sn + (int64_t)h * a.o_sh + cc * 8;
        const int4 *pp = reinterpret_cast<const int4 *>(pr + rr * SKP);
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        for (int j0 = 0; j0 < SKP; j0 += GB) {
            int4 e2[GB / 2];
#pragma unroll
            for (int u = 0; u < GB / 2; ++u) e2[u] = pp[j0 / 2 + u];
            typename IO::raw8 fr[GB];
#pragma unroll
            for (int u = 0; u < GB / 2; ++u) {
                fr[2 * u] = IO::load_raw(V + (uint32_t)e2[u].x);
                fr[2 * u + 1] = IO::load_raw(V + (uint32_t)e2[u].z);
            }
#pragma unroll
            for (int u = 0; u < GB; ++u) {
                float fv[8];
                IO::cvt(fr[u], fv);
                const float wv = __int_as_float(u & 1 ? e2[u / 2].w : e2[u / 2].y);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] += wv * fv[e];
            }
        }
        IO::store8(O, acc);
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

template <typename T, int KT>
aff_status launch_deform_k(const aff_deform_args &a, const Segs &segs, const DLayout &dl, void *ws, hipStream_t s) {
    BArgs ba{};
    char *w = static_cast<char *>(ws);
    ba.segs = segs;
    ba.wl = dl.g;
    ba.ws = ws;
    ba.fp = reinterpret_cast<FineParams *>(w + dl.fparams);
    ba.fcell = reinterpret_cast<int2 *>(w + dl.fcell);
    ba.counter = reinterpret_cast<int *>(w + dl.counter);
    ba.pool = reinterpret_cast<CandBlock *>(w + dl.pool);
    for (int l = 0; l <= segs.L; ++l) {
        ba.fc_off[l] = dl.fc_off[l];
        ba.tile_off[l] = dl.tile_off[l];
        if (l < segs.L) ba.fcmax[l] = dl.fcmax[l];
    }
    ba.fc_per_b = dl.fc_per_b;
    ba.pool_per_b = dl.pool_per_b;
    ba.tt_per_b = dl.tt_per_b;
    ba.K = a.K;
    const aff_status st = grid::launch_build(a.kv_pos, a.kp_sb, a.kp_sn, a.B, segs, ws, s, ZeroSpan{ba.counter, a.B});
    if (st != AFF_OK) return st;
    hipLaunchKernelGGL((cand_build_kernel<KT>), dim3((unsigned)(a.B * dl.tt_per_b)), dim3(CB), 0, s, ba);

    CArgs ka{};
    ka.a = a;
    ka.segs = segs;
    ka.wl = dl.g;
    ka.ws = ws;
    ka.fp = ba.fp;
    ka.fcell = ba.fcell;
    ka.pool = ba.pool;
    for (int l = 0; l <= segs.L; ++l) ka.fc_off[l] = dl.fc_off[l];
    ka.fc_per_b = dl.fc_per_b;
    ka.pool_per_b = dl.pool_per_b;
    ka.osz = a.off_dtype == AFF_F32 ? 4 : 2;
    ka.asz = a.attn_dtype == AFF_F32 ? 4 : 2;
    int pl = 0;
    while ((1 << pl) < a.P) ++pl;
    ka.pl_log2 = pl;
    const int RW = 64 >> pl;
    const int SKP = (a.L * a.P * a.K + PAIR_GROUP - 1) / PAIR_GROUP * PAIR_GROUP;
    const size_t per_wave = sizeof(int2) * (size_t)RW * SKP;  // <= 32 KB (L * P <= 32, K <= 8)
    const int nwv = per_wave * 4 <= 65536 ? 4 : 1;
    const int64_t rows = (int64_t)a.B * a.Nq * a.H;
    const int64_t blocks = (rows + (int64_t)RW * nwv - 1) / ((int64_t)RW * nwv);
    const dim3 grid((unsigned)blocks), block(64 * nwv);
    if (a.L == 1)
        hipLaunchKernelGGL((deform_cand_kernel<T, KT, 1>), grid, block, per_wave * nwv, s, ka);
    else if (a.L <= 4)
        hipLaunchKernelGGL((deform_cand_kernel<T, KT, 4>), grid, block, per_wave * nwv, s, ka);
    else
        hipLaunchKernelGGL((deform_cand_kernel<T, KT, 8>), grid, block, per_wave * nwv, s, ka);
    return check_launch("aff_deform_fwd");
}

template <typename T>
aff_status launch_deform(const aff_deform_args &a, const Segs &segs, const DLayout &dl, void *ws, hipStream_t s) {
    if (a.K <= 3) return launch_deform_k<T, 3>(a, segs, dl, ws, s);
    if (a.K <= 4) return launch_deform_k<T, 4>(a, segs, dl, ws, s);
    return launch_deform_k<T, KMAX>(a, segs, dl, ws, s);
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
    return deform::d_layout(args->B, segs, args->K).total;
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
    AFF_CHECK_ARG((int64_t)a.B * a.Nq * a.H < ((int64_t)1 << 31), "aff_deform_fwd: B*Nq*H must be below 2^31");
    AFF_CHECK_ARG(a.query_pos && a.kv_pos && a.offsets && a.attn && a.values && a.out && a.power,
                  "aff_deform_fwd: NULL pointer");
    AFF_CHECK_ARG(a.off_dtype >= 0 && a.off_dtype <= 2 && a.attn_dtype >= 0 && a.attn_dtype <= 2,
                  "aff_deform_fwd: offset/attention dtype");
    const int esz = a.dtype == AFF_F32 ? 4 : 2;
    for (int64_t s : {a.v_sb, a.v_sn, a.v_sh, a.o_sb, a.o_sn, a.o_sh})
        AFF_CHECK_ARG((s * esz) % 16 == 0, "aff_deform_fwd: value/output strides must keep 16-byte rows");
    AFF_CHECK_ARG(deform::a16(a.values) && deform::a16(a.out), "aff_deform_fwd: values/out must be 16-byte aligned");
    // offset pairs are read as dwords: 4-byte aligned pairs
    const int osz = a.off_dtype == AFF_F32 ? 4 : 2;
    AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(a.offsets) & 3) == 0 &&
                      ((a.off_sb | a.off_sn | a.off_sh) * osz) % 4 == 0,
                  "aff_deform_fwd: offsets must be 4-byte aligned with even strides");
    AFF_CHECK_ARG((int64_t)(a.level_start[a.L] > 0 ? a.level_start[a.L] - 1 : 0) * a.v_sn + (int64_t)(a.H - 1) * a.v_sh +
                      a.C < ((int64_t)1 << 31),
                  "aff_deform_fwd: one image's values must span fewer than 2^31 elements");
    if (a.L * a.P > 32) return fail(AFF_ERR_UNSUPPORTED, "aff_deform_fwd: L*P=%d exceeds 32 samples per head", a.L * a.P);
    const deform::DLayout dl = deform::d_layout(a.B, segs, a.K);
    if (!ws || ws_bytes < dl.total)
        return fail(AFF_ERR_WORKSPACE, "aff_deform_fwd: workspace of %zu bytes needed, got %zu", dl.total, ws_bytes);
    AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(ws) & 255) == 0, "aff_deform_fwd: workspace must be 256-byte aligned");
    AFF_CHECK_ARG((int64_t)a.B * dl.tt_per_b < ((int64_t)1 << 31), "aff_deform_fwd: too many build tiles");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (a.dtype == AFF_F32) return deform::launch_deform<float>(a, segs, dl, ws, s);
    if (a.dtype == AFF_BF16) return deform::launch_deform<bf16_t>(a, segs, dl, ws, s);
    return deform::launch_deform<f16_t>(a, segs, dl, ws, s);
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
