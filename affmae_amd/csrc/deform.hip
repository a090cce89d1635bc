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

#include <limits.h>

namespace aff {
namespace deform {

using namespace grid;

constexpr int THREADS = 256;
constexpr int KMAX = 8;    // neighbours per sample
constexpr int NB = 8;
constexpr int WMAX = 2048;        // window points held in LDS (all levels)
constexpr int WROWS = THREADS;    // window cell rows (all levels), one thread each while sizing
constexpr int WCMAX = 2048;       // window cell-offset entries (all levels)

__device__ __forceinline__ int64_t load_index(const void *p, int is_i64, int64_t i) {
    return is_i64 ? static_cast<const int64_t *>(p)[i] : int64_t(static_cast<const int32_t *>(p)[i]);
}

struct KArgs {
    aff_deform_args a;
    Segs segs;
    WsLayout wl;
    const void *ws;
};

// Order-preserving map of a float onto int (for min / max through integer LDS ops).
__device__ __forceinline__ int ford(float f) {
    const int i = __float_as_int(f);
    return i ^ ((i >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float fdeord(int i) { return __int_as_float(i ^ ((i >> 31) & 0x7fffffff)); }

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

// Window of one level staged in LDS: cells [wx0, wx1] x [wy0, wy1] of the
// level's grid; wcs[(cy - wy0) * (wx1 - wx0 + 2) + (cx - wx0)] is the LDS
// slot of the first point of cell (cx, cy).
struct LevelWin {
    int wx0, wy0, wx1, wy1, wcs;  // wcs: offset of this level's table in s_wcs
};

// Exact K nearest points (keys (d2, row) ascending, KT slots, the first keff
// meaningful) of (qx, qy) among the points of one level, visiting the cells
// meeting the disk d2 <= U from the LDS window; U grows until the keff-th key
// lies inside the visited disk.  Returns false when the disk leaves the
// window (the caller then searches the global grid).
template <int KT>
__device__ __forceinline__ bool topk_window(const GridParams &p, const LevelWin &w, const int *wcs,
                                            const float4 *pts, float qx, float qy, float U, int keff,
                                            uint64_t (&keys)[KT]) {
    const float slack = query_slack(p, qx, qy);
    for (int it = 0; it < 32; ++it) {
#pragma unroll
        for (int i = 0; i < KT; ++i) keys[i] = ~0ull;
        const float r = __builtin_amdgcn_sqrtf(U) * 1.00002f + slack;
        const int cy0 = cell_coord(qy - r, p.y0, p.inv_h, p.gy), cy1 = cell_coord(qy + r, p.y0, p.inv_h, p.gy);
        if (cy0 < w.wy0 || cy1 > w.wy1) return false;
        const int wxp = w.wx1 - w.wx0 + 2;
        for (int cy = cy0; cy <= cy1; ++cy) {
            const float rlo = p.y0 + float(cy) * p.h, rhi = rlo + p.h;
            const float dy = fmaxf(0.f, fmaxf(rlo - qy, qy - rhi) - slack);
            const float w2 = r * r - dy * dy;
            if (!(w2 >= 0.f)) continue;
            const float hw = __builtin_amdgcn_sqrtf(w2) * 1.00002f + slack;
            const int cx0 = cell_coord(qx - hw, p.x0, p.inv_h, p.gx), cx1 = cell_coord(qx + hw, p.x0, p.inv_h, p.gx);
            if (cx0 < w.wx0 || cx1 > w.wx1) return false;
            const int *row = wcs + w.wcs + (cy - w.wy0) * wxp - w.wx0;
            const int beg = row[cx0], end = row[cx1 + 1];
            for (int t = beg; t < end; t += 2) {  // two points per step (the array has a spare entry)
                const float4 a0 = pts[t], a1 = pts[t + 1];
                const uint64_t k0 = make_key(dist2(a0.x, a0.y, qx, qy), __float_as_int(a0.z));
                const uint64_t k1 = make_key(dist2(a1.x, a1.y, qx, qy), __float_as_int(a1.z));
                topk_insert<KT>(keys, k0);
                if (t + 1 < end) topk_insert<KT>(keys, k1);
            }
        }
        const uint64_t kth = keys[keff - 1 < KT ? keff - 1 : KT - 1];
        if (kth != ~0ull && key_d2(kth) <= U) return true;
        U = fmaxf(U * 2.f, kth != ~0ull ? key_d2(kth) : U);
        if (!(U < INFINITY)) return false;
    }
    return false;
}

// The same search over the global grid (always completes).
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

// SPR: lanes per (b, q, h) row = next power of two >= L * P.  KT: neighbour
// slots per sample (>= K).  A workgroup takes PASSES blocks of R = 256 / SPR
// consecutive rows: one LDS window (the cells of every level around all of
// its samples) serves all of them.
constexpr int PASSES = 8;

template <typename T, int SPR, int KT>
__global__ __launch_bounds__(THREADS) void deform_fwd_kernel(const KArgs ka) {
    using IO = ElemIO<T>;
    constexpr int R = THREADS / SPR;             // rows per pass
    __shared__ __align__(16) float4 s_pts[WMAX + 1];
    __shared__ int s_wcs[WCMAX];
    __shared__ int s_rb[WROWS + 1];              // LDS slot of each window row's first point
    __shared__ int s_gb[WROWS];                  // its slot in the level's cell-ordered array
    __shared__ int s_bb[AFF_DEFORM_MAX_LEVELS][4];
    __shared__ LevelWin s_lw[AFF_DEFORM_MAX_LEVELS];
    __shared__ int s_lrows[AFF_DEFORM_MAX_LEVELS], s_lcells[AFF_DEFORM_MAX_LEVELS];
    __shared__ GridParams s_gp[AFF_DEFORM_MAX_LEVELS];  // level grids of image b0
    __shared__ float s_rho[AFF_DEFORM_MAX_LEVELS];      // their mean point densities
    __shared__ int s_meta[4];                    // rows, cell entries, -, window ok
    __shared__ int s_wsum[THREADS / 64];
    __shared__ int s_row[R][SPR * KT];
    __shared__ float s_w[R][SPR * KT];

    const aff_deform_args &a = ka.a;
    const int tid = threadIdx.x;
    const int r = tid / SPR, t = tid % SPR;
    const int S = a.L * a.P, K = a.K, L = a.L;
    const int64_t total = (int64_t)a.B * a.Nq * a.H;
    const int64_t rowA = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * R * PASSES;
    const int b0 = int(rowA / ((int64_t)a.Nq * a.H));  // the window's image: that of the first row
    const int l = t < S ? t / a.P : 0;                 // level of this lane's sample (every pass)

    // ---- this lane's sample in pass ps: location and attention weight
    auto load_sample = [&](int ps, float &sx, float &sy, float &aw, int &bs) {
        const int64_t row = rowA + ps * R + r;
        sx = sy = aw = 0.f;
        bs = -1;
        if (row < total && t < S) {
            const uint32_t rw = uint32_t(row);  // the host keeps B * Nq * H below 2^31
            const int h = int(rw % uint32_t(a.H));
            const uint32_t bq = rw / uint32_t(a.H);
            const int q = int(bq % uint32_t(a.Nq)), b = int(bq / uint32_t(a.Nq));
            const float qx = a.query_pos[(int64_t)b * a.qp_sb + (int64_t)q * a.qp_sn];
            const float qy = a.query_pos[(int64_t)b * a.qp_sb + (int64_t)q * a.qp_sn + 1];
            const int64_t ob = (int64_t)b * a.off_sb + (int64_t)q * a.off_sn + (int64_t)h * a.off_sh + (int64_t)t * 2;
            sx = qx + load_any(a.offsets, a.off_dtype, ob);
            sy = qy + load_any(a.offsets, a.off_dtype, ob + 1);
            aw = load_any(a.attn, a.attn_dtype, (int64_t)b * a.at_sb + (int64_t)q * a.at_sn + (int64_t)h * a.at_sh + t);
            bs = b;
        }
    };
    // ---- bounding box of this lane's samples over all passes (image b0)
    int bmin = INT_MAX, bmaxx = INT_MIN, bminy = INT_MAX, bmaxy = INT_MIN;
#pragma unroll 1
    for (int ps = 0; ps < PASSES; ++ps) {
        float sx, sy, aw;
        int bs;
        load_sample(ps, sx, sy, aw, bs);
        if (bs == b0) {
            bmin = min(bmin, ford(sx));
            bmaxx = max(bmaxx, ford(sx));
            bminy = min(bminy, ford(sy));
            bmaxy = max(bmaxy, ford(sy));
        }
    }
    if (tid < AFF_DEFORM_MAX_LEVELS * 4) (&s_bb[0][0])[tid] = (tid & 1) ? INT_MIN : INT_MAX;
    __syncthreads();
    // ---- per-level bounding box of the workgroup's samples (image b0)
    if (bmin != INT_MAX) {
        atomicMin(&s_bb[l][0], bmin);
        atomicMax(&s_bb[l][1], bmaxx);
        atomicMin(&s_bb[l][2], bminy);
        atomicMax(&s_bb[l][3], bmaxy);
    }
    __syncthreads();

    // ---- window rectangles (thread lv per level): the box widened by 2 x the
    // radius holding K + 4 points at the level's mean density; a lane whose search
    // disk still leaves the window searches the global grid instead
    if (tid < L) {
        const int lv = tid;
        const SegView g = seg_view(ka.ws, ka.wl, ka.segs, b0, lv);
        const GridParams &p = g.p;
        LevelWin w{0, 0, -1, -1, 0};
        const float area = float(p.gx) * float(p.gy) * p.h * p.h;
        const float rho = float(g.n) / fmaxf(area, 1e-30f);
        s_gp[lv] = p;
        s_rho[lv] = rho;
        if (s_bb[lv][0] != INT_MAX && g.n > 0) {
            const float m = 2.f * sqrtf(float(K + 4) / (3.14159265f * rho));
            w.wx0 = cell_coord(fdeord(s_bb[lv][0]) - m, p.x0, p.inv_h, p.gx);
            w.wx1 = cell_coord(fdeord(s_bb[lv][1]) + m, p.x0, p.inv_h, p.gx);
            w.wy0 = cell_coord(fdeord(s_bb[lv][2]) - m, p.y0, p.inv_h, p.gy);
            w.wy1 = cell_coord(fdeord(s_bb[lv][3]) + m, p.y0, p.inv_h, p.gy);
        }
        s_lw[lv] = w;
        s_lrows[lv] = w.wy1 - w.wy0 + 1;
        s_lcells[lv] = (w.wx1 - w.wx0 + 2) * (w.wy1 - w.wy0 + 1);
    }
    __syncthreads();
    if (tid == 0) {
        int rows = 0, cells = 0;
        for (int lv = 0; lv < L; ++lv) {
            s_lw[lv].wcs = cells;
            rows += s_lrows[lv];
            cells += s_lcells[lv];
        }
        s_meta[0] = rows;
        s_meta[1] = cells;
        s_meta[3] = (rows <= WROWS && cells <= WCMAX) ? 1 : 0;
    }
    __syncthreads();
    bool win = s_meta[3] != 0;
    if (win) {
        // window row `tid`: its level, its cell range in the level's cell-ordered array
        const int nrows = s_meta[0];
        int cnt = 0, gb = 0;
        if (tid < nrows) {
            int lv = 0, base = 0;
            while (tid >= base + s_lrows[lv]) base += s_lrows[lv++];
            const LevelWin w = s_lw[lv];
            const SegView g = seg_view(ka.ws, ka.wl, ka.segs, b0, lv);
            const int *crow = g.cs + (w.wy0 + tid - base) * g.p.gx;
            gb = crow[w.wx0];
            cnt = crow[w.wx1 + 1] - gb;
        }
        // block exclusive scan of the row counts
        const int lane = tid & 63, wid = tid >> 6;
        int incl = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o, 64);
            if (lane >= o) incl += y;
        }
        if (lane == 63) s_wsum[wid] = incl;
        __syncthreads();
        int off = 0;
        for (int i = 0; i < wid; ++i) off += s_wsum[i];
        const int total_pts = s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
        if (tid < nrows) {
            s_rb[tid] = off + incl - cnt;
            s_gb[tid] = gb;
        }
        if (tid == 0) s_rb[nrows] = total_pts;
        win = total_pts <= WMAX;
        __syncthreads();
        if (win) {
            // cell-offset tables, then the points (x, y, row in the image's level
            // concatenation, as the global grid stores them)
            const int ncells = s_meta[1];
            for (int e = tid; e < ncells; e += THREADS) {
                int lv = 0, rbase = 0;
                while (lv + 1 < L && e >= s_lw[lv + 1].wcs) rbase += s_lrows[lv++];
                const LevelWin &w = s_lw[lv];
                const int wxp = w.wx1 - w.wx0 + 2, el = e - w.wcs;
                const int rr = el / wxp, c = el - rr * wxp;
                const SegView g = seg_view(ka.ws, ka.wl, ka.segs, b0, lv);
                s_wcs[e] = s_rb[rbase + rr] + g.cs[(w.wy0 + rr) * g.p.gx + w.wx0 + c] - s_gb[rbase + rr];
            }
            for (int e = tid; e < total_pts; e += THREADS) {
                int lo = 0, hi = nrows - 1;  // last row with s_rb[row] <= e
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (s_rb[mid] <= e) lo = mid; else hi = mid - 1;
                }
                int lv = 0, base = 0;
                while (lo >= base + s_lrows[lv]) base += s_lrows[lv++];
                const SegView g = seg_view(ka.ws, ka.wl, ka.segs, b0, lv);
                s_pts[e] = g.P[s_gb[lo] + (e - s_rb[lo])];
            }
            if (tid == 0) s_pts[total_pts] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
    }
    const float pw = *a.power;
    float nsx, nsy, naw;  // the next pass's sample, loaded one pass ahead
    int nbs;
    load_sample(0, nsx, nsy, naw, nbs);

#pragma unroll 1
    for (int ps = 0; ps < PASSES; ++ps) {
    const float sx = nsx, sy = nsy, aw = naw;
    if (ps + 1 < PASSES) load_sample(ps + 1, nsx, nsy, naw, nbs);
    const int64_t row = rowA + ps * R + r;
    const bool active = row < total;
    const uint32_t rw = active ? uint32_t(row) : 0u;
    const int h = int(rw % uint32_t(a.H));
    const uint32_t bq = rw / uint32_t(a.H);
    const int q = int(bq % uint32_t(a.Nq)), b = int(bq / uint32_t(a.Nq));
    const bool samp = active && t < S;

    // ---- phase A: one lane per sample; pairs of sample t occupy slots [t * K, t * K + K)
    for (int j = 0; j < KT; ++j) {
        s_row[r][t * KT + j] = -1;
        s_w[r][t * KT + j] = 0.f;
    }
    __syncthreads();
    if (samp) {
        const int nl = ka.segs.start[l + 1] - ka.segs.start[l];
        const int keff = min(K, nl);
        uint64_t keys[KT];
#pragma unroll
        for (int j = 0; j < KT; ++j) keys[j] = ~0ull;
        if (keff > 0) {
            // initial radius^2: the disk holding keff + 4 points at the level's mean density
            bool done = false;
            if (win && b == b0 && keff < nl) {
                const float U0 = fmaxf(float(keff + 4) / (3.14159265f * s_rho[l]), 1e-30f);
                done = topk_window<KT>(s_gp[l], s_lw[l], s_wcs, s_pts, sx, sy, U0, keff, keys);
            }
            if (!done) {
                const SegView g = seg_view(ka.ws, ka.wl, ka.segs, b, l);
                const float area = float(g.p.gx) * float(g.p.gy) * g.p.h * g.p.h;
                const float rho = float(g.n) / fmaxf(area, 1e-30f);
                const float U0 = keff >= g.n ? INFINITY : fmaxf(float(keff + 4) / (3.14159265f * rho), 1e-30f);
                topk_global<KT>(g, sx, sy, U0, keff, keys);
            }
        }
        float wj[KT];
        float wsum = 0.f;
        if (a.mode == AFF_DEFORM_SHEPARD) {
            const float p = fmaxf(pw, 1e-6f);
            float lg[KT], mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < KT; ++j) {
                lg[j] = j < keff ? -p * (sqrtf(key_d2(keys[j])) + 1e-6f) : -INFINITY;
                mx = fmaxf(mx, lg[j]);
            }
#pragma unroll
            for (int j = 0; j < KT; ++j) {
                wj[j] = j < keff ? __expf(lg[j] - mx) : 0.f;
                wsum += wj[j];
            }
            wsum += 1e-8f;
        } else {
#pragma unroll
            for (int j = 0; j < KT; ++j) {
                wj[j] = j < keff ? 1.f / (__powf(key_d2(keys[j]), pw) + 1e-10f) : 0.f;
                wsum += wj[j];
            }
            wsum += 1e-12f;
        }
        const float inv = 1.f / wsum;
        const int64_t kb = ((row * a.L * a.P) + t) * K;   // [B, Nq, H, L, P, K]
        const int lstart = ka.segs.start[l];
#pragma unroll
        for (int j = 0; j < KT; ++j) {
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
    // pair subset sg = t / CG (pairs sg, sg + NSG, ...), then the subsets are
    // summed across lanes.  Pairs of sample s sit at [s * K, s * K + K) within
    // the row's staging (K <= KT).
    const int C = a.C, CG = C / 8;
    const int npair = S * K;
    const T *V = static_cast<const T *>(a.values) + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh;
    T *O = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)q * a.o_sn + (int64_t)h * a.o_sh;
    if (SPR >= CG) {
        const int NSG = SPR / CG;
        const int cc = t % CG, sg = t / CG;
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        if (active) {
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
        // sum the NSG subsets: lanes cc, cc + CG, ... of the row
        for (int o = CG; o < SPR; o <<= 1)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o, 64);
        if (active && sg == 0) IO::store8(O + cc * 8, acc);
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
    __syncthreads();  // the next pass rewrites s_row / s_w
    }  // passes
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
aff_status launch_deform_k(const KArgs &ka, int spr, hipStream_t s) {
    const int64_t rows = (int64_t)ka.a.B * ka.a.Nq * ka.a.H;
    const int64_t per_block = (THREADS / spr) * PASSES;
    const int64_t blocks = (rows + per_block - 1) / per_block;
    switch (spr) {
#define DF_CASE(S) case S: hipLaunchKernelGGL((deform_fwd_kernel<T, S, KT>), dim3((unsigned)blocks), dim3(THREADS), 0, s, ka); break;
        DF_CASE(1) DF_CASE(2) DF_CASE(4) DF_CASE(8) DF_CASE(16) DF_CASE(32)
#undef DF_CASE
        default: return fail(AFF_ERR_UNSUPPORTED, "aff_deform_fwd: L*P=%d exceeds 32", spr);
    }
    return check_launch("aff_deform_fwd");
}

template <typename T>
aff_status launch_deform(const KArgs &ka, int spr, hipStream_t s) {
    const int K = ka.a.K;
    if (K <= 3) return launch_deform_k<T, 3>(ka, spr, s);
    if (K <= 4) return launch_deform_k<T, 4>(ka, spr, s);
    return launch_deform_k<T, KMAX>(ka, spr, s);
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
    AFF_CHECK_ARG((int64_t)a.B * a.Nq * a.H < ((int64_t)1 << 31), "aff_deform_fwd: B*Nq*H must be below 2^31");
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
