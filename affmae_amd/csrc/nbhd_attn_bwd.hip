// Neighbourhood (cluster) attention, backward, for gfx950.
//
// Gradient semantics follow the reference's backward kernels
// (src/layers/kernels/local_attn.py:350-606): Delta = rowsum(out * dout),
// p_j = exp(s_j - lse), dS_j = p_j (<dout, v_j> - Delta), dq = scale * sum
// dS_j k_j (plus the blank token's term), dk[idx_j] += scale dS_j q,
// dv[idx_j] += p_j dout, dbias = dS, and the blank tokens' gradients summed
// over every row of their head.  Masked and out-of-range neighbours receive
// no gradient.
//
// The reference scatters dk / dv / dbias / dblank with floating-point
// atomics, so its sums depend on scheduling.  Here every scattered sum is a
// gather in a fixed order instead:
//
// 1. bwd_rows_kernel, one (b, h, n) row per D/8 lanes: recomputes s_j, p_j,
//    <dout, v_j> and dS_j, writes dq, and keeps p_j and dS_j of every
//    (row, neighbour) pair (and the blank token's p and dS per row).
// 2. The pairs are bucketed by the key row they point at (bucket.hpp): keys
//    (b * N + idx_j) with payload (b * N + n) * M + j, stably sorted, so each
//    key row's incoming pairs are listed in (b, n, j) order.
// 3. bwd_keys_kernel, one (b, h, key row) per D/8 lanes: walks its bucket in
//    order and accumulates dk = scale * sum dS q_n and dv = sum p dout_n.
// 4. Bias modes 2 / 4: the pairs are bucketed again by table row and
//    table_grad_kernel sums each row's dS per head (one wave per row, lanes
//    over the bucket in order, a fixed butterfly across lanes).
// 5. The blank tokens: per-chunk partial sums over rows in a fixed order,
//    then the chunks summed in order.
#include "common.hpp"
#include "nbhd_attn_common.hpp"

#include "bucket.hpp"

namespace aff {
namespace attn_bwd {

using attn::MASKED_LOGIT;
using attn::load_index;
using attn::pe_from_coords;

constexpr int THREADS = 256;
constexpr int NB = 8;          // neighbours per block in the row pass
constexpr int KB = 4;          // bucket entries in flight per key row
constexpr int BLANK_CHUNKS = 256;

// ------------------------------------------------------------- row pass --
template <typename T, int D, int BIAS>
__global__ __launch_bounds__(THREADS) void bwd_rows_kernel(const aff_nbhd_attn_bwd_args g, float *P, float *dS,
                                                           float *pb_row, float *dsb_row) {
    using IO = ElemIO<T>;
    constexpr int LPR = D / 8;
    constexpr int ROWS = THREADS / LPR;
    const aff_nbhd_attn_args &a = g.fwd;
    const int sub = threadIdx.x % LPR;
    const int64_t row = (int64_t)blockIdx.x * ROWS + threadIdx.x / LPR;
    const int64_t total = (int64_t)a.B * a.H * a.N;
    if (row >= total) return;  // whole lane groups leave together
    const int N = a.N, M = a.M, H = a.H;
    const int n = int(row % N);
    const int64_t bh = row / N;
    const int b = int(bh / H), h = int(bh % H);

    const T *Kb = static_cast<const T *>(a.k) + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh + sub * 8;
    const T *Vb = static_cast<const T *>(a.v) + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh + sub * 8;
    float qv[8], dov[8], ov[8];
    IO::load8(static_cast<const T *>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)n * a.q_sn + sub * 8, qv);
    IO::load8(static_cast<const T *>(g.dout) + (int64_t)b * g.do_sb + (int64_t)h * g.do_sh + (int64_t)n * g.do_sn + sub * 8,
              dov);
    IO::load8(static_cast<const T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)n * a.o_sn + sub * 8, ov);
    const float lse = a.lse[row];
    float dl = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) dl += dov[i] * ov[i];
    const float delta = group_sum<LPR>(dl);

    const int64_t mi_row = (int64_t)b * a.mi_sb + (int64_t)n * a.mi_sn;
    const uint8_t *mrow = a.mask ? a.mask + (int64_t)b * a.mask_sb + (int64_t)h * a.mask_sh + (int64_t)n * a.mask_sn
                                 : nullptr;
    float pqx = 0.f, pqy = 0.f;
    const float *pos_b = nullptr;
    const float relW = float(a.rel_width), relT = float(2 * a.rel_width + 1);
    if constexpr (BIAS == 4) {
        pos_b = a.pos + (int64_t)b * a.pos_sb;
        pqx = pos_b[(int64_t)n * a.pos_sn];
        pqy = pos_b[(int64_t)n * a.pos_sn + 1];
    }
    float *Prow = P + row * M, *dSrow = dS + row * M;

    float dq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dq[i] = 0.f;

    for (int j0 = 0; j0 < M; j0 += NB) {
        int64_t idx[NB];
        bool valid[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int j = j0 + u;
            const bool live = j < M;
            idx[u] = live ? load_index(a.member_idx, a.idx_is_i64, mi_row + j) : 0;
            bool ok = live && idx[u] >= 0 && idx[u] < N;
            if (mrow && live) ok = ok && (mrow[j] != 0);
            valid[u] = ok;
        }
        typename IO::raw8 kr[NB], vr[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int64_t r = valid[u] ? idx[u] : 0;
            kr[u] = IO::load_raw(Kb + r * a.k_sn);
            vr[u] = IO::load_raw(Vb + r * a.v_sn);
        }
        float bias[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            bias[u] = 0.f;
            if (!valid[u]) continue;
            const int j = j0 + u;
            if constexpr (BIAS == 1) {
                bias[u] = load_any(a.bias, a.bias_dtype,
                                   (int64_t)b * a.bias_sb + (int64_t)h * a.bias_sh + (int64_t)n * a.bias_sn + j);
            } else if constexpr (BIAS == 2) {
                const int64_t pe = load_index(a.pe_idx, a.pe_is_i64, (int64_t)b * a.pe_sb + (int64_t)n * a.pe_sn + j);
                if (pe >= 0 && pe < a.table_rows) bias[u] = load_any(a.table, a.table_dtype, pe * H + h);
            } else if constexpr (BIAS == 4) {
                const float mx = pos_b[idx[u] * a.pos_sn], my = pos_b[idx[u] * a.pos_sn + 1];
                const int64_t pe = pe_from_coords(pqx, pqy, mx, my, relW, relT);
                if (pe >= 0 && pe < a.table_rows) bias[u] = load_any(a.table, a.table_dtype, pe * H + h);
            }
        }
        float pj[NB], dsj[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            float kf[8], vf[8];
            IO::cvt(kr[u], kf);
            IO::cvt(vr[u], vf);
            float sd = 0.f, pd = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                sd += qv[i] * kf[i];
                pd += dov[i] * vf[i];
            }
            sd = group_sum<LPR>(sd);
            pd = group_sum<LPR>(pd);
            const float s = sd * a.scale + bias[u];
            const float p = valid[u] ? __expf(s - lse) : 0.f;
            const float ds = p * (pd - delta);
            pj[u] = p;
            dsj[u] = ds;
#pragma unroll
            for (int i = 0; i < 8; ++i) dq[i] += ds * kf[i];
        }
        // every lane of the row holds the pair values: lane sub stores entries u = sub, sub + LPR, ...
#pragma unroll
        for (int u = 0; u < NB; ++u)
            if (u % LPR == sub && j0 + u < M) {
                Prow[j0 + u] = pj[u];
                dSrow[j0 + u] = dsj[u];
            }
    }

    if (a.blank_k) {
        float bk[8], bv[8];
        IO::load8(static_cast<const T *>(a.blank_k) + h * D + sub * 8, bk);
        IO::load8(static_cast<const T *>(a.blank_v) + h * D + sub * 8, bv);
        float sd = 0.f, pd = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            sd += qv[i] * bk[i];
            pd += dov[i] * bv[i];
        }
        sd = group_sum<LPR>(sd);
        pd = group_sum<LPR>(pd);
        const float p = __expf(sd * a.scale - lse);
        const float ds = p * (pd - delta);
#pragma unroll
        for (int i = 0; i < 8; ++i) dq[i] += ds * bk[i];
        if (sub == 0) {
            pb_row[row] = p;
            dsb_row[row] = ds;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) dq[i] *= a.scale;
    IO::store8(static_cast<T *>(g.dq) + (int64_t)b * g.dq_sb + (int64_t)h * g.dq_sh + (int64_t)n * g.dq_sn + sub * 8, dq);
}

// --------------------------------------------------------- bucket index --
// Key of every (b, n, j) pair: b * N + idx (pairs a shared mask or the index
// range excludes get the sentinel B * N); payload (b * N + n) * M + j.
__global__ __launch_bounds__(THREADS) void kv_keys_kernel(const aff_nbhd_attn_args a, unsigned *keys, int *vals) {
    const int64_t e = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.N * a.M;
    if (e >= total) return;
    const int M = a.M, N = a.N;
    const int j = int(e % M);
    const int64_t bn = e / M;
    const int n = int(bn % N), b = int(bn / N);
    const int64_t idx = load_index(a.member_idx, a.idx_is_i64, (int64_t)b * a.mi_sb + (int64_t)n * a.mi_sn + j);
    bool ok = idx >= 0 && idx < N;
    if (ok && a.mask && a.mask_sh == 0) ok = a.mask[(int64_t)b * a.mask_sb + (int64_t)n * a.mask_sn + j] != 0;
    keys[e] = ok ? unsigned(b * (int64_t)N + idx) : unsigned(a.B * N);
    vals[e] = int(e);
}

// Key of every pair for the table gradient: the table row the forward read
// (bias mode 2: pe_idx; mode 4: from the coordinates), or the sentinel
// table_rows for pairs without one.
template <int BIAS>
__global__ __launch_bounds__(THREADS) void table_keys_kernel(const aff_nbhd_attn_args a, unsigned *keys, int *vals) {
    const int64_t e = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.N * a.M;
    if (e >= total) return;
    const int M = a.M, N = a.N;
    const int j = int(e % M);
    const int64_t bn = e / M;
    const int n = int(bn % N), b = int(bn / N);
    const int64_t idx = load_index(a.member_idx, a.idx_is_i64, (int64_t)b * a.mi_sb + (int64_t)n * a.mi_sn + j);
    bool ok = idx >= 0 && idx < N;
    if (ok && a.mask && a.mask_sh == 0) ok = a.mask[(int64_t)b * a.mask_sb + (int64_t)n * a.mask_sn + j] != 0;
    int64_t pe = -1;
    if (ok) {
        if constexpr (BIAS == 2) {
            pe = load_index(a.pe_idx, a.pe_is_i64, (int64_t)b * a.pe_sb + (int64_t)n * a.pe_sn + j);
        } else {
            const float *pos_b = a.pos + (int64_t)b * a.pos_sb;
            pe = pe_from_coords(pos_b[(int64_t)n * a.pos_sn], pos_b[(int64_t)n * a.pos_sn + 1], pos_b[idx * a.pos_sn],
                                pos_b[idx * a.pos_sn + 1], float(a.rel_width), float(2 * a.rel_width + 1));
        }
    }
    const bool in = pe >= 0 && pe < a.table_rows;
    keys[e] = in ? unsigned(pe) : unsigned(a.table_rows);
    vals[e] = int(e);
}

// ------------------------------------------------------------- key pass --
template <typename T, int D>
__global__ __launch_bounds__(THREADS) void bwd_keys_kernel(const aff_nbhd_attn_bwd_args g, const float *P,
                                                           const float *dS, const int *vals, const int *off) {
    using IO = ElemIO<T>;
    constexpr int LPR = D / 8;
    constexpr int ROWS = THREADS / LPR;
    const aff_nbhd_attn_args &a = g.fwd;
    const int sub = threadIdx.x % LPR;
    const int64_t row = (int64_t)blockIdx.x * ROWS + threadIdx.x / LPR;
    const int64_t total = (int64_t)a.B * a.H * a.N;
    if (row >= total) return;
    const int N = a.N, M = a.M, H = a.H;
    const int r = int(row % N);
    const int64_t bh = row / N;
    const int b = int(bh / H), h = int(bh % H);
    const int64_t NM = (int64_t)N * M;
    // pair (n, j) of image b, head h: element (b * H + h) * N * M + n * M + j of P / dS;
    // payload v = (b * N + n) * M + j, so the element is v + ((b * H + h) - b) * N * M
    const int64_t shift = ((int64_t)b * H + h - b) * NM;
    const T *Qb = static_cast<const T *>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + sub * 8;
    const T *Db = static_cast<const T *>(g.dout) + (int64_t)b * g.do_sb + (int64_t)h * g.do_sh + sub * 8;
    const int lo = off[(int64_t)b * N + r], hi = off[(int64_t)b * N + r + 1];

    float dk[8], dv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dk[i] = dv[i] = 0.f;
    for (int e0 = lo; e0 < hi; e0 += KB) {
        int64_t pr[KB];
        int nn[KB];
        bool live[KB];
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            live[u] = e0 + u < hi;
            const int64_t v = live[u] ? vals[e0 + u] : (int64_t)b * NM;
            pr[u] = v + shift;
            nn[u] = int(v / M - (int64_t)b * N);
        }
        typename IO::raw8 qr[KB], dr[KB];
        float ds[KB], p[KB];
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            qr[u] = IO::load_raw(Qb + (int64_t)nn[u] * a.q_sn);
            dr[u] = IO::load_raw(Db + (int64_t)nn[u] * g.do_sn);
            ds[u] = live[u] ? dS[pr[u]] : 0.f;
            p[u] = live[u] ? P[pr[u]] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            float qf[8], df[8];
            IO::cvt(qr[u], qf);
            IO::cvt(dr[u], df);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                dk[i] += ds[u] * qf[i];
                dv[i] += p[u] * df[i];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) dk[i] *= a.scale;
    IO::store8(static_cast<T *>(g.dk) + (int64_t)b * g.dk_sb + (int64_t)h * g.dk_sh + (int64_t)r * g.dk_sn + sub * 8, dk);
    IO::store8(static_cast<T *>(g.dv) + (int64_t)b * g.dv_sb + (int64_t)h * g.dv_sh + (int64_t)r * g.dv_sn + sub * 8, dv);
}

// ----------------------------------------------------------- table rows --
// dtable[t, h] = sum of dS over the pairs of bucket t, head h: one wave per
// table row, lane l sums entries l, l + 64, ... in order, then a fixed xor
// butterfly across the 64 lanes.
__global__ __launch_bounds__(THREADS) void table_grad_kernel(const aff_nbhd_attn_args a, const float *dS,
                                                             const int *vals, const int *off, float *dtable) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6);
    if (t >= a.table_rows) return;  // whole waves leave together
    const int lo = off[t], hi = off[t + 1];
    const int H = a.H;
    const int64_t NM = (int64_t)a.N * a.M;
    for (int h = 0; h < H; ++h) {
        float s = 0.f;
        for (int e = lo + lane; e < hi; e += 64) {
            const int64_t v = vals[e];
            const int64_t b = v / NM;
            s += dS[v + (b * H + h - b) * NM];
        }
        s = group_sum<64>(s);
        if (lane == 0) dtable[t * H + h] = s;
    }
}

// ----------------------------------------------------------- blank tokens --
// Partial sums over chunk c of the B * N rows of head h:
//   part_k[c, h, :] = sum dS_blank q,  part_v[c, h, :] = sum p_blank dout.
template <typename T, int D>
__global__ __launch_bounds__(THREADS) void blank_partial_kernel(const aff_nbhd_attn_bwd_args g, const float *pb_row,
                                                                const float *dsb_row, float *part_k, float *part_v) {
    using IO = ElemIO<T>;
    constexpr int LPR = D / 8;
    constexpr int RPB = THREADS / LPR;
    const aff_nbhd_attn_args &a = g.fwd;
    const int c = blockIdx.x, h = blockIdx.y;
    const int sub = threadIdx.x % LPR, slot = threadIdx.x / LPR;
    const int64_t rows = (int64_t)a.B * a.N;
    const int64_t per = (rows + gridDim.x - 1) / gridDim.x;
    const int64_t r0 = (int64_t)c * per, r1 = r0 + per < rows ? r0 + per : rows;
    float ak[8], av[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ak[i] = av[i] = 0.f;
    for (int64_t r = r0 + slot; r < r1; r += RPB) {
        const int b = int(r / a.N), n = int(r % a.N);
        const int64_t row = ((int64_t)b * a.H + h) * a.N + n;
        float qf[8], df[8];
        IO::load8(static_cast<const T *>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)n * a.q_sn + sub * 8, qf);
        IO::load8(static_cast<const T *>(g.dout) + (int64_t)b * g.do_sb + (int64_t)h * g.do_sh + (int64_t)n * g.do_sn +
                      sub * 8,
                  df);
        const float ds = dsb_row[row], p = pb_row[row];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ak[i] += ds * qf[i];
            av[i] += p * df[i];
        }
    }
    // fixed-order tree over the RPB row slots
    __shared__ float red[2][RPB][D + 1];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        red[0][slot][sub * 8 + i] = ak[i];
        red[1][slot][sub * 8 + i] = av[i];
    }
    __syncthreads();
    for (int w = RPB / 2; w > 0; w >>= 1) {
        for (int e = threadIdx.x; e < 2 * w * D; e += THREADS) {
            const int kv = e / (w * D), rem = e % (w * D), s = rem / D, d = rem % D;
            red[kv][s][d] += red[kv][s + w][d];
        }
        __syncthreads();
    }
    for (int d = threadIdx.x; d < D; d += THREADS) {
        part_k[((int64_t)c * a.H + h) * D + d] = red[0][0][d];
        part_v[((int64_t)c * a.H + h) * D + d] = red[1][0][d];
    }
}

__global__ __launch_bounds__(THREADS) void blank_final_kernel(const float *part_k, const float *part_v, int chunks,
                                                              int HD, float scale, float *dbk, float *dbv) {
    const int e = blockIdx.x * THREADS + threadIdx.x;
    if (e >= HD) return;
    float sk = 0.f, sv = 0.f;
    for (int c = 0; c < chunks; ++c) {
        sk += part_k[(int64_t)c * HD + e];
        sv += part_v[(int64_t)c * HD + e];
    }
    dbk[e] = sk * scale;
    dbv[e] = sv;
}

// ------------------------------------------------------------------ host --
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct BwdLayout {
    size_t P, dS, pb, dsb, keys_in, vals_in, keys_out, vals_out, off_kv, off_tab, temp, part_k, part_v, total;
    size_t temp_bytes;
};

inline bool wants_table(const aff_nbhd_attn_bwd_args &g) {
    return g.dtable != nullptr && (g.fwd.bias_mode == 2 || g.fwd.bias_mode == 4);
}

inline BwdLayout layout(const aff_nbhd_attn_bwd_args &g) {
    const aff_nbhd_attn_args &a = g.fwd;
    const int64_t rows = (int64_t)a.B * a.H * a.N, pairs_h = rows * a.M, pairs = (int64_t)a.B * a.N * a.M;
    BwdLayout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = align256(off + bytes);
        return at;
    };
    L.P = take(sizeof(float) * pairs_h);
    L.dS = g.dbias ? 0 : take(sizeof(float) * pairs_h);
    L.pb = a.blank_k ? take(sizeof(float) * rows) : 0;
    L.dsb = a.blank_k ? take(sizeof(float) * rows) : 0;
    L.keys_in = take(sizeof(unsigned) * pairs);
    L.vals_in = take(sizeof(int) * pairs);
    L.keys_out = take(sizeof(unsigned) * pairs);
    L.vals_out = take(sizeof(int) * pairs);
    L.off_kv = take(sizeof(int) * ((int64_t)a.B * a.N + 1));
    L.off_tab = wants_table(g) ? take(sizeof(int) * (a.table_rows + 1)) : 0;
    size_t tb = bucket::sort_temp_bytes(pairs, bucket::key_bits((int64_t)a.B * a.N));
    if (wants_table(g)) {
        const size_t t2 = bucket::sort_temp_bytes(pairs, bucket::key_bits(a.table_rows));
        tb = t2 > tb ? t2 : tb;
    }
    L.temp_bytes = tb;
    L.temp = take(tb);
    L.part_k = a.blank_k ? take(sizeof(float) * BLANK_CHUNKS * a.H * a.D) : 0;
    L.part_v = a.blank_k ? take(sizeof(float) * BLANK_CHUNKS * a.H * a.D) : 0;
    L.total = off;
    return L;
}

using RowsFn = void (*)(const aff_nbhd_attn_bwd_args, float *, float *, float *, float *);
using KeysFn = void (*)(const aff_nbhd_attn_bwd_args, const float *, const float *, const int *, const int *);
using BlankFn = void (*)(const aff_nbhd_attn_bwd_args, const float *, const float *, float *, float *);

template <typename T, int D>
RowsFn pick_rows_bias(int mode) {
    switch (mode) {
        case 0: return bwd_rows_kernel<T, D, 0>;
        case 1: return bwd_rows_kernel<T, D, 1>;
        case 2: return bwd_rows_kernel<T, D, 2>;
        default: return bwd_rows_kernel<T, D, 4>;
    }
}

template <typename T>
RowsFn pick_rows(int D, int mode) {
    switch (D) {
        case 8: return pick_rows_bias<T, 8>(mode);
        case 16: return pick_rows_bias<T, 16>(mode);
        case 32: return pick_rows_bias<T, 32>(mode);
        case 64: return pick_rows_bias<T, 64>(mode);
        default: return pick_rows_bias<T, 128>(mode);
    }
}

template <typename T>
KeysFn pick_keys(int D) {
    switch (D) {
        case 8: return bwd_keys_kernel<T, 8>;
        case 16: return bwd_keys_kernel<T, 16>;
        case 32: return bwd_keys_kernel<T, 32>;
        case 64: return bwd_keys_kernel<T, 64>;
        default: return bwd_keys_kernel<T, 128>;
    }
}

template <typename T>
BlankFn pick_blank(int D) {
    switch (D) {
        case 8: return blank_partial_kernel<T, 8>;
        case 16: return blank_partial_kernel<T, 16>;
        case 32: return blank_partial_kernel<T, 32>;
        case 64: return blank_partial_kernel<T, 64>;
        default: return blank_partial_kernel<T, 128>;
    }
}

template <typename Fn>
Fn by_dtype(int dtype, Fn f32, Fn bf16, Fn f16) {
    return dtype == AFF_F32 ? f32 : dtype == AFF_BF16 ? bf16 : f16;
}

inline unsigned blocks_for(int64_t items, int per_block) { return (unsigned)((items + per_block - 1) / per_block); }

}  // namespace attn_bwd
}  // namespace aff

using namespace aff;

extern "C" size_t aff_nbhd_attn_bwd_workspace_bytes(const aff_nbhd_attn_bwd_args *args) {
    if (args == nullptr || (int64_t)args->fwd.B * args->fwd.H * args->fwd.N == 0) return 0;
    return attn_bwd::layout(*args).total;
}

extern "C" aff_status aff_nbhd_attn_bwd(const aff_nbhd_attn_bwd_args *args, aff_stream_t stream) {
    using namespace attn_bwd;
    AFF_CHECK_ARG(args != nullptr, "aff_nbhd_attn_bwd: NULL args");
    const aff_nbhd_attn_bwd_args &g = *args;
    const aff_nbhd_attn_args &a = g.fwd;
    AFF_CHECK_ARG(a.B >= 0 && a.H >= 1 && a.N >= 0 && a.M >= 0, "aff_nbhd_attn_bwd: bad sizes B=%d H=%d N=%d M=%d",
                  a.B, a.H, a.N, a.M);
    if (a.D != 8 && a.D != 16 && a.D != 32 && a.D != 64 && a.D != 128)
        return fail(AFF_ERR_UNSUPPORTED, "aff_nbhd_attn_bwd: head_dim %d not compiled (8/16/32/64/128)", a.D);
    if (a.dtype != AFF_F32 && a.dtype != AFF_F16 && a.dtype != AFF_BF16)
        return fail(AFF_ERR_UNSUPPORTED, "aff_nbhd_attn_bwd: dtype %d", a.dtype);
    AFF_CHECK_ARG(a.bias_mode >= 0 && a.bias_mode <= 4, "aff_nbhd_attn_bwd: bias_mode %d", a.bias_mode);
    if (a.bias_mode == 3)
        return fail(AFF_ERR_UNSUPPORTED, "aff_nbhd_attn_bwd: the continuous bias (mode 3) has no backward here");
    AFF_CHECK_ARG(g.dtable == nullptr || a.bias_mode == 2 || a.bias_mode == 4,
                  "aff_nbhd_attn_bwd: dtable needs bias mode 2 or 4");
    AFF_CHECK_ARG((g.dblank_k == nullptr) == (g.dblank_v == nullptr),
                  "aff_nbhd_attn_bwd: dblank_k and dblank_v must both be set or both NULL");
    AFF_CHECK_ARG((a.blank_k == nullptr) == (a.blank_v == nullptr),
                  "aff_nbhd_attn_bwd: blank_k and blank_v must both be set or both NULL");
    AFF_CHECK_ARG(a.blank_k == nullptr || g.dblank_k != nullptr,
                  "aff_nbhd_attn_bwd: the forward had blank tokens: dblank_k / dblank_v are required");
    const int64_t rows = (int64_t)a.B * a.H * a.N;
    if (rows == 0) return AFF_OK;
    AFF_CHECK_ARG(a.q && a.k && a.v && a.out && a.lse && g.dout && g.dq && g.dk && g.dv,
                  "aff_nbhd_attn_bwd: NULL q/k/v/out/lse/dout/dq/dk/dv");
    AFF_CHECK_ARG(a.M == 0 || a.member_idx, "aff_nbhd_attn_bwd: NULL member_idx");
    AFF_CHECK_ARG((int64_t)a.B * a.N * a.M < ((int64_t)1 << 31) && rows * a.M < ((int64_t)1 << 40),
                  "aff_nbhd_attn_bwd: problem too large (B*N*M must fit in 31 bits)");
    const int esz = a.dtype == AFF_F32 ? 4 : 2;
    const int64_t st[] = {a.q_sb, a.q_sh, a.q_sn, a.k_sb, a.k_sh, a.k_sn, a.v_sb, a.v_sh, a.v_sn,
                          a.o_sb, a.o_sh, a.o_sn, g.do_sb, g.do_sh, g.do_sn, g.dq_sb, g.dq_sh, g.dq_sn,
                          g.dk_sb, g.dk_sh, g.dk_sn, g.dv_sb, g.dv_sh, g.dv_sn};
    for (int64_t s : st) AFF_CHECK_ARG((s * esz) % 16 == 0, "aff_nbhd_attn_bwd: strides must keep 16-byte row alignment");
    auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    AFF_CHECK_ARG(al16(a.q) && al16(a.k) && al16(a.v) && al16(a.out) && al16(g.dout) && al16(g.dq) && al16(g.dk) &&
                      al16(g.dv) && (!a.blank_k || (al16(a.blank_k) && al16(a.blank_v))),
                  "aff_nbhd_attn_bwd: tensors must be 16-byte aligned");
    if (a.bias_mode == 1) AFF_CHECK_ARG(a.bias != nullptr, "aff_nbhd_attn_bwd: bias_mode 1 needs bias");
    if (a.bias_mode == 2) AFF_CHECK_ARG(a.pe_idx && a.table, "aff_nbhd_attn_bwd: bias_mode 2 needs pe_idx and table");
    if (a.bias_mode == 4) AFF_CHECK_ARG(a.pos && a.table, "aff_nbhd_attn_bwd: bias_mode 4 needs pos and table");

    const BwdLayout L = layout(g);
    AFF_CHECK_ARG((reinterpret_cast<uintptr_t>(g.ws) & 255) == 0, "aff_nbhd_attn_bwd: workspace must be 256-byte aligned");
    if (g.ws == nullptr || g.ws_bytes < L.total)
        return fail(AFF_ERR_WORKSPACE, "aff_nbhd_attn_bwd: workspace of %zu bytes needed, got %zu", L.total,
                    g.ws ? g.ws_bytes : (size_t)0);
    char *ws = static_cast<char *>(g.ws);
    float *P = reinterpret_cast<float *>(ws + L.P);
    float *dS = g.dbias ? g.dbias : reinterpret_cast<float *>(ws + L.dS);
    float *pb = a.blank_k ? reinterpret_cast<float *>(ws + L.pb) : nullptr;
    float *dsb = a.blank_k ? reinterpret_cast<float *>(ws + L.dsb) : nullptr;
    unsigned *keys_in = reinterpret_cast<unsigned *>(ws + L.keys_in), *keys_out = reinterpret_cast<unsigned *>(ws + L.keys_out);
    int *vals_in = reinterpret_cast<int *>(ws + L.vals_in), *vals_out = reinterpret_cast<int *>(ws + L.vals_out);
    int *off_kv = reinterpret_cast<int *>(ws + L.off_kv);
    hipStream_t hs = static_cast<hipStream_t>(stream);
    const int dt = a.dtype, D = a.D;
    const int lpr = D / 8, rows_per_block = THREADS / lpr;
    const int64_t pairs = (int64_t)a.B * a.N * a.M;

    // 1. rows: dq, P, dS, blank terms
    const RowsFn rows_fn = by_dtype(dt, pick_rows<float>(D, a.bias_mode), pick_rows<bf16_t>(D, a.bias_mode),
                                    pick_rows<f16_t>(D, a.bias_mode));
    hipLaunchKernelGGL(rows_fn, dim3(blocks_for(rows, rows_per_block)), dim3(THREADS), 0, hs, g, P, dS, pb, dsb);
    aff_status s = check_launch("aff_nbhd_attn_bwd (rows)");
    if (s != AFF_OK) return s;

    // 2. bucket the pairs by key row, 3. dk / dv
    const int nkv = a.B * a.N;
    if (pairs > 0) {
        hipLaunchKernelGGL(kv_keys_kernel, dim3(blocks_for(pairs, THREADS)), dim3(THREADS), 0, hs, a, keys_in, vals_in);
        if ((s = check_launch("aff_nbhd_attn_bwd (keys)")) != AFF_OK) return s;
    }
    if ((s = bucket::sort_and_offsets(keys_in, vals_in, keys_out, vals_out, pairs, nkv, ws + L.temp, L.temp_bytes,
                                      off_kv, hs)) != AFF_OK)
        return s;
    const KeysFn keys_fn = by_dtype(dt, pick_keys<float>(D), pick_keys<bf16_t>(D), pick_keys<f16_t>(D));
    hipLaunchKernelGGL(keys_fn, dim3(blocks_for(rows, rows_per_block)), dim3(THREADS), 0, hs, g, P, dS, vals_out, off_kv);
    if ((s = check_launch("aff_nbhd_attn_bwd (key rows)")) != AFF_OK) return s;

    // 4. table rows
    if (wants_table(g)) {
        int *off_tab = reinterpret_cast<int *>(ws + L.off_tab);
        const int tr = (int)a.table_rows;
        if (pairs > 0) {
            hipLaunchKernelGGL(a.bias_mode == 2 ? table_keys_kernel<2> : table_keys_kernel<4>,
                               dim3(blocks_for(pairs, THREADS)), dim3(THREADS), 0, hs, a, keys_in, vals_in);
            if ((s = check_launch("aff_nbhd_attn_bwd (table keys)")) != AFF_OK) return s;
        }
        if ((s = bucket::sort_and_offsets(keys_in, vals_in, keys_out, vals_out, pairs, tr, ws + L.temp, L.temp_bytes,
                                          off_tab, hs)) != AFF_OK)
            return s;
        hipLaunchKernelGGL(table_grad_kernel, dim3(blocks_for(tr, THREADS / 64)), dim3(THREADS), 0, hs, a, dS, vals_out,
                           off_tab, g.dtable);
        if ((s = check_launch("aff_nbhd_attn_bwd (table rows)")) != AFF_OK) return s;
    }

    // 5. blank tokens
    if (a.blank_k) {
        float *pk = reinterpret_cast<float *>(ws + L.part_k), *pv = reinterpret_cast<float *>(ws + L.part_v);
        const BlankFn bf = by_dtype(dt, pick_blank<float>(D), pick_blank<bf16_t>(D), pick_blank<f16_t>(D));
        hipLaunchKernelGGL(bf, dim3(BLANK_CHUNKS, a.H), dim3(THREADS), 0, hs, g, pb, dsb, pk, pv);
        if ((s = check_launch("aff_nbhd_attn_bwd (blank partials)")) != AFF_OK) return s;
        hipLaunchKernelGGL(blank_final_kernel, dim3(blocks_for((int64_t)a.H * D, THREADS)), dim3(THREADS), 0, hs, pk, pv,
                           BLANK_CHUNKS, a.H * D, a.scale, g.dblank_k, g.dblank_v);
        if ((s = check_launch("aff_nbhd_attn_bwd (blank)")) != AFF_OK) return s;
    }
    return AFF_OK;
}
