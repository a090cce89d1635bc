// Neighbourhood (cluster) flash attention, forward, for gfx950.
//
// Semantics: _nbhood_attn_fwd / _update_online_softmax_block in the
// reference (src/layers/kernels/local_attn.py:80-116, 119-215, 224-340):
// masked neighbours take the logit -1e11 and a zero value row, the per-head
// blank token joins the softmax after the neighbours, the running maximum
// starts at -1e11 and LSE = m + log(l + 1e-12).
//
// Two kernels implement it; the host picks the first that takes the call.
//
// nbhd_attn_wave_kernel (bf16 / fp16, head_dim 32, M <= 64, any H and bias
// mode): one workgroup per (32-query tile, head group), one wave per head;
// described where it is defined.
//
// nbhd_attn_fwd_kernel (every dtype and head_dim, the rest): D/8 lanes own one
// (b, h, n) row (8 channels each).  Neighbours are consumed 8 at a time:
// indices, mask, bias and 16 K/V row pieces are loaded before use, then one
// online-softmax rescale is applied per block.
//
// Both kernels swizzle their block order so each XCD walks a contiguous
// range of images and keeps that image's K/V planes in its own L2.
#include "common.hpp"
#include "nbhd_attn_common.hpp"

#include <limits.h>

#include <algorithm>

namespace aff {
namespace attn {

constexpr int THREADS = 256;

// ------------------------------------------------------------------------
// Per-row routine: LPR = D/8 aligned lanes compute one (b, h, n) output row,
// NB neighbours per online-softmax block.
// ------------------------------------------------------------------------
template <typename T, int D, int BIAS, int NB>
__device__ __forceinline__ void attend_row(const aff_nbhd_attn_args &a, int b, int h, int n, int sub) {
    using IO = ElemIO<T>;
    constexpr int LPR = D / 8;
    const int N = a.N, M = a.M, H = a.H;

    const T *Kb = static_cast<const T *>(a.k) + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh + sub * 8;
    const T *Vb = static_cast<const T *>(a.v) + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh + sub * 8;

    float qv[8];
    IO::load8(static_cast<const T *>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                  (int64_t)n * a.q_sn + sub * 8,
              qv);
#pragma unroll
    for (int i = 0; i < 8; ++i) qv[i] *= a.scale;

    const int64_t mi_row = (int64_t)b * a.mi_sb + (int64_t)n * a.mi_sn;
    const uint8_t *mrow = a.mask ? a.mask + (int64_t)b * a.mask_sb + (int64_t)h * a.mask_sh +
                                       (int64_t)n * a.mask_sn
                                 : nullptr;

    // coordinate-bias constants (modes 3 and 4)
    float pqx = 0.f, pqy = 0.f, pw[5] = {0, 0, 0, 0, 0}, pb = 0.f;
    const float *pos_b = nullptr;
    const float relW = float(a.rel_width), relT = float(2 * a.rel_width + 1);
    if constexpr (BIAS == 3 || BIAS == 4) {
        pos_b = a.pos + (int64_t)b * a.pos_sb;
        pqx = pos_b[(int64_t)n * a.pos_sn];
        pqy = pos_b[(int64_t)n * a.pos_sn + 1];
    }
    if constexpr (BIAS == 3) {
#pragma unroll
        for (int f = 0; f < 5; ++f) pw[f] = a.pos_w[h * 5 + f];
        pb = a.pos_b[h];
    }

    float m = MASKED_LOGIT, l = 0.f;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;

    for (int j0 = 0; j0 < M; j0 += NB) {
        int64_t idx[NB];
        bool valid[NB], live[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int j = j0 + u;
            live[u] = j < M;
            idx[u] = live[u] ? load_index(a.member_idx, a.idx_is_i64, mi_row + j) : 0;
            bool ok = live[u] && idx[u] >= 0 && idx[u] < N;
            if (mrow && live[u]) ok = ok && (mrow[j] != 0);
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
                                   (int64_t)b * a.bias_sb + (int64_t)h * a.bias_sh +
                                       (int64_t)n * a.bias_sn + j);
            } else if constexpr (BIAS == 2) {
                const int64_t pe =
                    load_index(a.pe_idx, a.pe_is_i64, (int64_t)b * a.pe_sb + (int64_t)n * a.pe_sn + j);
                if (pe >= 0 && pe < a.table_rows) bias[u] = load_any(a.table, a.table_dtype, pe * H + h);
            } else if constexpr (BIAS == 3) {
                const float mx = pos_b[idx[u] * a.pos_sn], my = pos_b[idx[u] * a.pos_sn + 1];
                bias[u] = cont_bias(pw, pb, mx - pqx, my - pqy);
            } else if constexpr (BIAS == 4) {
                const float mx = pos_b[idx[u] * a.pos_sn], my = pos_b[idx[u] * a.pos_sn + 1];
                const int64_t pe = pe_from_coords(pqx, pqy, mx, my, relW, relT);
                if (pe >= 0 && pe < a.table_rows) bias[u] = load_any(a.table, a.table_dtype, pe * H + h);
            }
        }
        float s[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            float kf[8];
            IO::cvt(kr[u], kf);
            float d = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) d += qv[i] * kf[i];
            d = group_sum<LPR>(d);
            s[u] = valid[u] ? d + bias[u] : (live[u] ? MASKED_LOGIT : -INFINITY);
        }
        float mb = s[0];
#pragma unroll
        for (int u = 1; u < NB; ++u) mb = fmaxf(mb, s[u]);
        const float mn = fmaxf(m, mb);
        const float alpha = __expf(m - mn);
        l *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] *= alpha;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const float pu = __expf(s[u] - mn);
            l += pu;
            if (valid[u]) {
                float vf[8];
                IO::cvt(vr[u], vf);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[i] += pu * vf[i];
            }
        }
        m = mn;
    }

    if (a.blank_k) {
        float bk[8], bv[8];
        IO::load8(static_cast<const T *>(a.blank_k) + h * D + sub * 8, bk);
        IO::load8(static_cast<const T *>(a.blank_v) + h * D + sub * 8, bv);
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) d += qv[i] * bk[i];
        const float sb = group_sum<LPR>(d);
        const float mn = fmaxf(m, sb);
        const float alpha = __expf(m - mn), pb_ = __expf(sb - mn);
        l = l * alpha + pb_;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = acc[i] * alpha + pb_ * bv[i];
        m = mn;
    }

    const float lse = m + __logf(l + 1e-12f);
    const float inv = 1.f / (l + 1e-12f);
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = acc[i] * inv;
    IO::store8(static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh +
                   (int64_t)n * a.o_sn + sub * 8,
               o);
    if (a.lse && sub == 0) a.lse[((int64_t)b * H + h) * N + n] = lse;
}

template <typename T, int D, int BIAS>
__global__ __launch_bounds__(THREADS) void nbhd_attn_fwd_kernel(const aff_nbhd_attn_args a) {
    constexpr int LPR = D / 8;
    constexpr int ROWS = THREADS / LPR;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int sub = threadIdx.x % LPR;
    const int64_t row = (int64_t)bid * ROWS + threadIdx.x / LPR;
    const int64_t total = (int64_t)a.B * a.H * a.N;
    if (row >= total) return;  // whole lane groups leave together
    const int n = int(row % a.N);
    const int64_t bh = row / a.N;
    attend_row<T, D, BIAS, 8>(a, int(bh / a.H), int(bh % a.H), n, sub);
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane 4a + b receives
// element b of the four 16-bit values addressed by lanes a, 4 + a, 8 + a and
// 12 + a (in that order).  With lane 4k + a pointing at row s_k, columns
// 4a .. 4a + 3 of a row-major 16-bit tile, lane n therefore holds column n of
// rows s_0 .. s_3: a column of the tile, as an MFMA operand wants it.
typedef short tr_v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) tr_v4s lds_tr_v4s;
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t *p) {
    const tr_v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_tr_v4s *)(p));
    return __builtin_bit_cast(uint2, v);
}

// Max / sum over each aligned group of 8 lanes: two quad butterflies, then
// the half-row mirror (lane i <-> 7 - i) folds the other quad in.
__device__ __forceinline__ float grp8_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    return fmaxf(v, dpp_mov<0x141>(v));
}
__device__ __forceinline__ float grp8_sum(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    return v + dpp_mov<0x141>(v);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma32;
template <> struct Mfma32<bf16_t> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    __device__ __forceinline__ static f32x16 mma(uint4 a, uint4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0,
                                                       0, 0);
    }
    // one v_cvt_pk_bf16_f32 (round to nearest even)
    __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, b2));
    }
    __device__ __forceinline__ static float to_f32(uint16_t x) { return bf16_to_f32(x); }
};
template <> struct Mfma32<f16_t> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    __device__ __forceinline__ static f32x16 mma(uint4 a, uint4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0,
                                                      0);
    }
    // one v_cvt_pk_f16_f32 (round to nearest even)
    __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, h2));
    }
    __device__ __forceinline__ static float to_f32(uint16_t x) { return float(__builtin_bit_cast(_Float16, x)); }
};

namespace wt {
constexpr int TQ = 32;            // queries per workgroup (the MFMA N dimension)
constexpr int HD = 32;            // head_dim
constexpr int UMAX = 224;         // union rows: 7 chunks of 32 (a 16-query half tile: 2 UMAX)
constexpr int WWORDS = 256;       // index-window bitmap words: windows up to 8192 indices
constexpr int MAXM = 64;          // neighbours per query
constexpr int LPQ = 8;            // set-up lanes per query
constexpr int RJ = MAXM / LPQ;    // set-up entries per lane: j = jl + 8 r
constexpr int NW = THREADS / 64;  // waves; wave w takes heads w, w + NW, ...
constexpr int PWP = UMAX + 4;     // pw row pitch (8-bit codes): 228-byte rows
constexpr int MAXH = 64;          // heads of this kernel
constexpr int MAXHM = 196;        // (M + 1) * HG of the per-neighbour bias store
constexpr int BMW = TQ * MAXHM;   // bias store: fp32 words
constexpr int VRP = HD;           // V chunk row pitch (16-bit): 64-byte rows
constexpr float LOG2E = 1.4426950408889634f;
static_assert(WWORDS == THREADS, "one bitmap word per thread");
static_assert(TQ * LPQ == THREADS, "one set-up lane group per query");
static_assert((TQ * PWP) % 16 == 0 && PWP % 4 == 0, "pw is cleared in 16-byte pieces, read in 4-byte ones");
static_assert(2 * UMAX + 4 <= 2 * PWP, "a half tile's code rows hold 2 UMAX slots");
static_assert(MAXM + 1 < 256, "a code is an entry number + 1 in 8 bits");
static_assert(TQ * (NW * HD + 8) * 2 <= BMW * 4, "the projection's output block fits in the bias store");
}  // namespace wt

// max / sum of v over lanes l and l ^ 32 (v_permlane32_swap exchanges the two halves)
__device__ __forceinline__ float pair_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The per-row routine over rows n0 .. n0 + nq - 1 of image b, every head, 4 lanes
// per row (head_dim 32), 4 neighbours per block so that its registers stay
// below the wave kernel's own.
template <typename T, int BIAS>
__device__ __forceinline__ void tile_rows(const aff_nbhd_attn_args &a, int b, int n0, int nq, int hb, int hn) {
    const int sub = threadIdx.x & 3, rr = threadIdx.x >> 2;
    for (int p = rr; p < nq * hn; p += THREADS / 4) {
        const int qq = p % nq, hd = hb + p / nq;
        if (n0 + qq < a.N) attend_row<T, 32, BIAS, 4>(a, b, hd, n0 + qq, sub);
    }
}

// Head phase of one wave over a 32-query tile whose union (U rows, ulist), codes (pw)
// and bias store (bm) are in LDS: heads h0, h0 + hstep, ... below hend.  bm holds a plane
// per head of the group, (M + 1) entries per query, entry 0 the -inf one; a (query, slot)
// code c (8 bits: 0 or neighbour entry + 1) puts head h's bias at entry c of the query's
// row in head h's plane.
// nm: masked (live) neighbours of this lane's query; vbuf: the wave's V chunk buffer.
//
// Per 32-slot chunk:
//   S^T (32 slots x 32 queries) = K_chunk Q^T       2 x v_mfma_f32_32x32x16
//   logits (log2 units) = S * scale * log2(e) + bias(pw) * log2(e)
//   online softmax per query: lane l and lane l ^ 32 hold the 16 + 16 slots
//   of query l & 31, so the chunk maximum is one permlane32 swap
//   O^T (32 channels x 32 queries) += V_chunk^T P^T    2 x v_mfma_f32_32x32x16
// P^T is the S result itself converted to 16 bits: the PV contraction takes
// its k index in the order the S result lays slots out in the lanes, and
// V^T is read in that same order from the chunk's V rows in LDS by
// ds_read_b64_tr_b16.  K and V rows are fetched one chunk ahead.
// STAGE: the normalised outputs of the lane (channels 8 j + 4 hh + i of query ql at
// yo[4 j + i]) stay in registers for the projection epilogue instead of going to out.
template <typename T, bool BLANK, bool STAGE = false>
__device__ __forceinline__ void wave_head_one(const aff_nbhd_attn_args &a, int b, int n0, int U, const int *ulist,
                                              const uint8_t *pw, const float *bm, float nm, uint16_t *vbuf, int h,
                                              int hbase, int HG, float *yo = nullptr, int qlo = 0, int qhi = wt::TQ,
                                              int pitch = wt::PWP) {
    using namespace wt;
    using MM = Mfma32<T>;
    const int lane = threadIdx.x & 63;
    const int N = a.N, H = a.H;
    auto rsrc = [](const void *p) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, -1, 0x00020000);
    };
    const int hh = lane >> 5, ql = lane & 31;
    const int nch = (U + 31) >> 5;
    const bool qout = n0 + ql < N && ql >= qlo && ql < qhi;  // rows this call stores
    const int qrow = min(n0 + ql, N - 1);
    const uint32_t ksn2 = uint32_t(a.k_sn * 2), vsn2 = uint32_t(a.v_sn * 2);  // < 2^24, host-checked
    const uint32_t qoff = uint32_t(qrow) * uint32_t(a.q_sn * 2) + 32 * hh;
    const float scale2 = a.scale * LOG2E;
    // transposing-read role: 16-lane group g reads channels 16 (g & 1) + (lane & 15)
    const int kk = (lane & 15) >> 2, aa = lane & 3, cg = 16 * ((lane >> 4) & 1);
    // code rows: one per query of [qlo, qhi), `pitch` bytes apart (other lanes read row 0)
    const uint8_t *pwrow = pw + (ql >= qlo && ql < qhi ? ql - qlo : 0) * pitch + 4 * hh;
    // V rows go through a 16-row buffer: rows 0..15 of the chunk, then rows 16..31
    const uint32_t vst0 = (lane >> 2) * VRP + (lane & 3) * 8;
    const uint16_t *vtr = vbuf + (4 * hh + kk) * VRP + cg + 4 * aa;
    // K row of this lane in chunk c: union slot 32 c + ql; V pieces p = lane + 64 i: row p >> 2, bytes 16 (p & 3)
    auto koff = [&](int c) {
        const int s = 32 * c + ql;
        return __umul24(uint32_t(ulist[s < U ? s : 0]), ksn2) + 32 * hh;
    };
    auto voff = [&](int c, int i) {
        const int s = 32 * c + 16 * i + (lane >> 2);
        return __umul24(uint32_t(ulist[s < U ? s : 0]), vsn2) + 16 * (lane & 3);
    };
    auto ld = [](__amdgpu_buffer_rsrc_t rs, uint32_t off) {
        return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(off), 0, 0));
    };

    {
        const auto rq = rsrc(static_cast<const char *>(a.q) + ((int64_t)b * a.q_sb + (int64_t)h * a.q_sh) * 2);
        const auto rk = rsrc(static_cast<const char *>(a.k) + ((int64_t)b * a.k_sb + (int64_t)h * a.k_sh) * 2);
        const auto rv = rsrc(static_cast<const char *>(a.v) + ((int64_t)b * a.v_sb + (int64_t)h * a.v_sh) * 2);
        // K/V registers of two chunks: chunk c + 1 loads while chunk c computes
        uint4 kA0 = make_uint4(0, 0, 0, 0), kA1 = kA0, vA0 = kA0, vA1 = kA0;
        uint4 kB0 = kA0, kB1 = kA0, vB0 = kA0, vB1 = kA0;
        auto fetch = [&](int c, uint4 &k0, uint4 &k1, uint4 &v0, uint4 &v1) {
            const uint32_t ko = koff(c);
            k0 = ld(rk, ko);
            k1 = ld(rk, ko + 16);
            v0 = ld(rv, voff(c, 0));
            v1 = ld(rv, voff(c, 1));
        };
        if (nch > 0) fetch(0, kA0, kA1, vA0, vA1);
        const uint4 q0 = ld(rq, qoff), q1 = ld(rq, qoff + 16);
        float m = MASKED_LOGIT * LOG2E;
        float sb = 0.f;
        if constexpr (BLANK) {
            const char *bkp = static_cast<const char *>(a.blank_k) + (h * HD + 16 * hh) * 2;
            const uint4 bk0 = *reinterpret_cast<const uint4 *>(bkp), bk1 = *reinterpret_cast<const uint4 *>(bkp + 16);
            const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            const uint32_t kw[8] = {bk0.x, bk0.y, bk0.z, bk0.w, bk1.x, bk1.y, bk1.z, bk1.w};
            float part = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                part += MM::to_f32(uint16_t(qw[e] & 0xffffu)) * MM::to_f32(uint16_t(kw[e] & 0xffffu)) +
                        MM::to_f32(uint16_t(qw[e] >> 16)) * MM::to_f32(uint16_t(kw[e] >> 16));
            sb = pair_sum(part) * scale2;
            m = fmaxf(m, sb);
        }
        // head-major planes [HG][TQ][M + 1]: the lanes of one wave (one head) spread over all banks
        const char *bmh = reinterpret_cast<const char *>(bm) + 4 * (((h - hbase) * TQ + ql) * (a.M + 1));
        float lp = 0.f;
        f32x16 O;
#pragma unroll
        for (int r = 0; r < 16; ++r) O[r] = 0.f;

        // LDS data of the lane's 16 slots (8 j + 4 hh + i of a chunk): the codes are read
        // one chunk ahead, the biases at the start of their chunk (read during the S
        // MFMAs; no bias registers are held across chunks)
        auto read_codes = [&](int c, uint32_t (&cw)[4]) {
#pragma unroll
            for (int j = 0; j < 4; ++j) cw[j] = *reinterpret_cast<const uint32_t *>(pwrow + 32 * c + 8 * j);
        };
        auto read_bias = [&](const uint32_t (&cw)[4], float (&bias)[16]) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t code = (cw[r >> 2] >> (8 * (r & 3))) & 0xffu;
                bias[r] = *reinterpret_cast<const float *>(bmh + 4 * code);
            }
        };
        uint32_t cwA[4], cwB[4];
        if (nch > 0) read_codes(0, cwA);

        // chunk c: K/V registers k0..v1, codes cc; the codes of chunk c + 1 go to cn
        auto chunk = [&](int c, const uint4 &k0, const uint4 &k1, const uint4 &v0, const uint4 &v1,
                         const uint32_t (&cc)[4], uint32_t (&cn)[4]) {
            // this chunk's V rows through the wave's 16-row buffer and their transposed
            // reads, rows 0..15 then 16..31 (a wave's LDS operations complete in order, so
            // each store follows the reads issued before it)
            uint2 vt[4];
            asm volatile("" ::: "memory");
            *reinterpret_cast<uint4 *>(vbuf + vst0) = v0;
            asm volatile("" ::: "memory");
            vt[0] = lds_read_tr16(vtr);
            vt[1] = lds_read_tr16(vtr + 8 * VRP);
            asm volatile("" ::: "memory");
            *reinterpret_cast<uint4 *>(vbuf + vst0) = v1;
            asm volatile("" ::: "memory");
            vt[2] = lds_read_tr16(vtr);
            vt[3] = lds_read_tr16(vtr + 8 * VRP);
            float bc[16];
            read_bias(cc, bc);
            read_codes(min(c + 1, nch - 1), cn);
            f32x16 S;
#pragma unroll
            for (int r = 0; r < 16; ++r) S[r] = 0.f;
            S = MM::mma(k0, q0, S);
            S = MM::mma(k1, q1, S);
            float x[16];
            float cm = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                x[r] = fmaf(S[r], scale2, bc[r]);
                cm = fmaxf(cm, x[r]);
            }
            // the running maximum moves only when a logit exceeds it by more than 8
            // (probabilities then stay below 2^8), so the rescale is rare
            const float cmp = pair_max(cm);
            if (__builtin_amdgcn_ballot_w64(cmp > m + 8.f) != 0) {
                const float mn = fmaxf(m, cmp);
                const float alpha = __builtin_amdgcn_exp2f(m - mn);
                m = mn;
                lp *= alpha;
#pragma unroll
                for (int r = 0; r < 16; ++r) O[r] *= alpha;
            }
            float ps = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                x[r] = __builtin_amdgcn_exp2f(x[r] - m);
                ps += x[r];
            }
            lp += ps;
#pragma unroll
            for (int mm = 0; mm < 2; ++mm) {
                const uint4 pb = make_uint4(MM::pack2(x[8 * mm + 0], x[8 * mm + 1]), MM::pack2(x[8 * mm + 2], x[8 * mm + 3]),
                                            MM::pack2(x[8 * mm + 4], x[8 * mm + 5]), MM::pack2(x[8 * mm + 6], x[8 * mm + 7]));
                O = MM::mma(make_uint4(vt[2 * mm].x, vt[2 * mm].y, vt[2 * mm + 1].x, vt[2 * mm + 1].y), pb, O);
            }
        };

        // The fetches are unconditional (past the last chunk they re-read it): a
        // conditional load would make the compiler wait for it before the current
        // chunk's MFMAs on every path, serialising load latency with compute.
        for (int c = 0; c < nch; c += 2) {
            fetch(min(c + 1, nch - 1), kB0, kB1, vB0, vB1);
            chunk(c, kA0, kA1, vA0, vA1, cwA, cwB);
            if (c + 1 >= nch) break;
            fetch(min(c + 2, nch - 1), kA0, kA1, vA0, vA1);
            chunk(c + 1, kB0, kB1, vB0, vB1, cwB, cwA);
        }

        // ---- normalise, blank value, store: channels 8 j + 4 hh + i of query ql
        const float pbl = BLANK ? __builtin_amdgcn_exp2f(sb - m) : 0.f;
        const float l = pair_sum(lp) + pbl + (nm > 0.f ? nm * __builtin_amdgcn_exp2f(MASKED_LOGIT * LOG2E - m) : 0.f);
        const float inv = __builtin_amdgcn_rcpf(l + 1e-12f);  // 1 ulp: outputs are 16-bit
        if constexpr (STAGE) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d0 = 8 * j + 4 * hh;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float y = O[4 * j + i];
                    if constexpr (BLANK) {
                        const uint16_t bv = *reinterpret_cast<const uint16_t *>(
                            static_cast<const char *>(a.blank_v) + (h * HD + d0 + i) * 2);
                        y += pbl * MM::to_f32(bv);
                    }
                    yo[4 * j + i] = y * inv;
                }
            }
            if (qout && a.lse && hh == 0)
                a.lse[((int64_t)b * H + h) * N + n0 + ql] = m * 0.6931471805599453f + __logf(l + 1e-12f);
        } else if (qout) {
            T *orow = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)(n0 + ql) * a.o_sn;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d0 = 8 * j + 4 * hh;
                float y[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) y[i] = O[4 * j + i];
                if constexpr (BLANK) {
                    const uint2 bv = *reinterpret_cast<const uint2 *>(static_cast<const char *>(a.blank_v) + (h * HD + d0) * 2);
                    y[0] += pbl * MM::to_f32(uint16_t(bv.x & 0xffffu));
                    y[1] += pbl * MM::to_f32(uint16_t(bv.x >> 16));
                    y[2] += pbl * MM::to_f32(uint16_t(bv.y & 0xffffu));
                    y[3] += pbl * MM::to_f32(uint16_t(bv.y >> 16));
                }
                *reinterpret_cast<uint2 *>(orow + d0) =
                    make_uint2(MM::pack2(y[0] * inv, y[1] * inv), MM::pack2(y[2] * inv, y[3] * inv));
            }
            if (a.lse && hh == 0) a.lse[((int64_t)b * H + h) * N + n0 + ql] = m * 0.6931471805599453f + __logf(l + 1e-12f);
        }
    }
}

// Heads h0, h0 + hstep, ... below hend, one after another (wave_head_one).
template <typename T, bool BLANK>
__device__ __forceinline__ void wave_heads(const aff_nbhd_attn_args &a, int b, int n0, int U, const int *ulist,
                                           const uint8_t *pw, const float *bm, float nm, uint16_t *vbuf, int h0,
                                           int hstep, int hend, int hbase, int HG, int qlo, int qhi, int pitch) {
    for (int h = h0; h < hend; h += hstep)
        wave_head_one<T, BLANK>(a, b, n0, U, ulist, pw, bm, nm, vbuf, h, hbase, HG, nullptr, qlo, qhi, pitch);
}

// The output projection fused into the wave kernel's epilogue (ClusterAttention's
// proj, reference attention.py:204-205): y = O W^T + b for the tile's 32 queries,
// with every head of the image in the workgroup (at most NW heads, one per wave).
struct ProjArgs {
    const void *w;   // [C, C] 16-bit (the attention dtype), row o = output channel o
    const float *b;  // [C] or NULL
};

// y^T (32 output channels x 32 queries) per MFMA block = W_block O^T; O is the
// tile's [32][C] 16-bit block in LDS (row pitch op), W rows from global memory.
template <typename T>
__device__ __forceinline__ void proj_epilogue(const aff_nbhd_attn_args &a, const ProjArgs &pj, int b, int n0,
                                              const uint16_t *otile, int op, int C) {
    using namespace wt;
    using MM = Mfma32<T>;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int hh = lane >> 5, ql = lane & 31;
    const int nblk = C / 32;
    for (int ob = w; ob < nblk; ob += NW) {
        f32x16 Y;
#pragma unroll
        for (int r = 0; r < 16; ++r) Y[r] = 0.f;
        const uint16_t *wrow = static_cast<const uint16_t *>(pj.w) + (int64_t)(32 * ob + ql) * C + 8 * hh;
        const uint16_t *orow = otile + ql * op + 8 * hh;
        for (int k0 = 0; k0 < C; k0 += 16) {
            const uint4 wa = *reinterpret_cast<const uint4 *>(wrow + k0);
            const uint4 ov = *reinterpret_cast<const uint4 *>(orow + k0);
            Y = MM::mma(wa, ov, Y);
        }
        if (n0 + ql < a.N) {
            T *yrow = static_cast<T *>(a.out) + (int64_t)b * a.o_sb + (int64_t)(n0 + ql) * a.o_sn + 32 * ob;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int o0 = 8 * j + 4 * hh;
                float y[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) y[i] = Y[4 * j + i] + (pj.b ? pj.b[32 * ob + o0 + i] : 0.f);
                *reinterpret_cast<uint2 *>(yrow + o0) = make_uint2(MM::pack2(y[0], y[1]), MM::pack2(y[2], y[3]));
            }
        }
    }
}

template <typename T, int BIAS, bool IDX64, bool BLANK, bool PROJ = false>
__global__ __launch_bounds__(THREADS, 4) void nbhd_attn_wave_kernel(const aff_nbhd_attn_args a, int HG,
                                                                    const ProjArgs pj) {
    using namespace wt;
    using MM = Mfma32<T>;
    // pw[q][slot]: 1 + the neighbour entry of query q whose row is union slot `slot`; 0
    // where the slot is not one of the query's neighbours
    __shared__ __align__(16) uint8_t pw[TQ * PWP];
    // bm: biases of this workgroup's head group, times log2(e): [HG][TQ][M + 1], entry 0
    // of each (head, query) -inf, entry 1 + j neighbour j.  The LDS of a workgroup stays under
    // 40 KB, so that four fit on a CU.
    __shared__ __align__(16) float bm[BMW];
    __shared__ int ulist[2 * UMAX];
    struct SetupLds {
        uint32_t bits[WWORDS];  // one bit per index of the window: a neighbour row
        uint32_t pref[WWORDS];  // union slots before each word
    };
    __shared__ __align__(16) union {
        SetupLds s;
        uint16_t vb[NW][16 * VRP];  // per-wave 16-row V buffer (head phase)
    } sh;
    __shared__ float nmq_s[TQ];
    __shared__ int red[4];  // 0 flagged, 1 repeated index, 2 U

    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);  // wave-uniform: heads index scalar buffers
    const int N = a.N, M = a.M, H = a.H;
    const int tiles = (N + TQ - 1) / TQ;
    // workgroup = (tile, head group): the groups of one tile are adjacent, so on one XCD
    const int ngroups = (H + HG - 1) / HG;
    const int wg = int(xcd_swizzle(blockIdx.x, gridDim.x));
    const int tile = wg / ngroups, hb = (wg % ngroups) * HG, hn = min(HG, H - hb);
    const int b = tile / tiles;
    const int n0 = (tile % tiles) * TQ;
    const int nr = (M + LPQ - 1) / LPQ;  // entries per set-up lane that exist (uniform)

    // One pass over the tile's queries [qlo, qhi); the other queries act as dead rows (no
    // entries, nothing stored).  With split set, a pass whose union is wider than UMAX
    // (the tile not flagged otherwise) stores nothing and returns true: the caller then
    // runs the two 16-query halves, each with the union of its own rows (up to 2 UMAX: its
    // 16 code rows take the 32 rows' space at twice the pitch), instead of the per-row
    // routine for all 32 (a half still wider runs the per-row routine).
    auto run = [&](const int qlo, const int qhi, const bool split) __attribute__((always_inline)) -> bool {
    // The lane's indices come from an opaque copy of the thread index in every pass, so
    // that the compiler recomputes their addresses instead of keeping one pass's values
    // live (spilled) into the next.
    int t = int(threadIdx.x);
    asm volatile("" : "+v"(t));
    const int lane = t & 63, q = t >> 3, jl = t & 7;
    const int n = n0 + q, nc = min(n, N - 1);
    const bool mine = q >= qlo && q < qhi;  // this lane's query belongs to the pass
    const bool qlive = n < N && mine;

    if (t < 4) red[t] = 0;
    // Table bias modes write the bias store only after the slots step, so their union flags
    // (a byte per window index, plain stores) live in its space until then; the other modes
    // write biases while loading the entries and set the union bits with LDS atomics.
    constexpr bool FLAGS = BIAS == 2 || BIAS == 4;
    static_assert(WWORDS * 32 <= BMW * 4, "the union flags fit in the bias store");
    uint8_t *flg = reinterpret_cast<uint8_t *>(bm);
    auto init_inf = [&]() {
        for (int i = t; i < TQ * HG; i += THREADS) bm[i * (M + 1)] = -INFINITY;  // (head, query) = (i / TQ, i % TQ)
    };
    if constexpr (FLAGS) {
        for (int i = t; i < WWORDS * 2; i += THREADS) reinterpret_cast<uint4 *>(flg)[i] = make_uint4(0, 0, 0, 0);
    } else {
        sh.s.bits[t] = 0u;  // WWORDS == THREADS
        init_inf();
    }
    for (int i = t; i < TQ * PWP / 16; i += THREADS) reinterpret_cast<uint4 *>(pw)[i] = make_uint4(0, 0, 0, 0);

    // ---- this lane's (query, neighbour) entries j = jl + 8 r.  Loads are unconditional
    // buffer loads at 32-bit offsets inside this image's planes (clamped to entry M - 1
    // and row nc; the host keeps the offsets below 2^31), validity is a select.
    auto rsrc = [](const void *p) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, -1, 0x00020000);
    };
    const int mlast = max(M - 1, 0);
    const auto r_mi = rsrc(static_cast<const char *>(a.member_idx) + (int64_t)b * a.mi_sb * (IDX64 ? 8 : 4));
    const uint32_t mi_off = uint32_t(nc) * uint32_t(a.mi_sn);
    int idx[RJ];
    bool use[RJ];
    int nmask = 0;
#pragma unroll
    for (int r = 0; r < RJ; ++r) {
        use[r] = false;
        idx[r] = nc;
        if (r >= nr) continue;
        const int j = jl + LPQ * r, jc = min(j, mlast);
        const bool live = qlive && j < M;
        bool ok;
        int ix;
        if constexpr (IDX64) {
            const auto v2 = __builtin_amdgcn_raw_buffer_load_b64(r_mi, int((mi_off + jc) * 8), 0, 0);
            const int64_t v = int64_t(uint64_t(v2[0]) | (uint64_t(v2[1]) << 32));
            ok = live && v >= 0 && v < N;
            ix = int(v);
        } else {
            const int v = int(__builtin_amdgcn_raw_buffer_load_b32(r_mi, int((mi_off + jc) * 4), 0, 0));
            ok = live && unsigned(v) < unsigned(N);
            ix = v;
        }
        if (a.mask) {
            const auto r_mk = rsrc(a.mask + (int64_t)b * a.mask_sb);
            ok = ok && __builtin_amdgcn_raw_buffer_load_b8(r_mk, int(uint32_t(nc) * uint32_t(a.mask_sn) + jc), 0, 0) != 0;
        }
        use[r] = ok;
        idx[r] = ok ? ix : nc;
        nmask += (live && !ok) ? 1 : 0;
    }

    // ---- biases of the entries, every head, times log2(e), for bm.  Table modes
    // (2, 4): the entries' table-row inputs (pe rows, or the neighbours' coordinates)
    // are loaded here and stay in flight through the union steps; the rows are read
    // and bm written after the slots (write_table_biases).  Modes 1 and 3 store at
    // once; mode 0 stores zeros.
    const int PL = TQ * (M + 1);             // bm words per head plane
    const int rowq_b = q * (M + 1) + 1;      // bm word of (q, j = 0) in head 0's plane
    const bool fast4 = (BIAS == 2 || BIAS == 4) && HG == 4 && H % 4 == 0 && a.table_dtype == AFF_F32;
    float2 gq[RJ];   // BIAS 4: neighbour coordinates
    int64_t prow[RJ];  // BIAS 2: pe rows
    float pqx = 0.f, pqy = 0.f;
    const float *pos_b = nullptr;
    if constexpr (BIAS == 3 || BIAS == 4) {
        pos_b = a.pos + (int64_t)b * a.pos_sb;
        const float2 pq = *reinterpret_cast<const float2 *>(pos_b + (int64_t)nc * a.pos_sn);
        pqx = pq.x;
        pqy = pq.y;
    }
    const int Tw = 2 * a.rel_width + 1;
#pragma unroll
    for (int r = 0; r < RJ; ++r) {
        gq[r] = make_float2(0.f, 0.f);
        prow[r] = -1;
        if (r >= nr) continue;
        const int j = jl + LPQ * r;
        if constexpr (BIAS == 4) {
            gq[r] = *reinterpret_cast<const float2 *>(pos_b + (int64_t)idx[r] * a.pos_sn);  // idx[r] is a valid row
        } else if constexpr (BIAS == 2) {
            if (use[r]) {
                const int64_t e = (int64_t)b * a.pe_sb + (int64_t)nc * a.pe_sn + j;
                prow[r] = a.pe_is_i64 ? static_cast<const int64_t *>(a.pe_idx)[e]
                                      : int64_t(static_cast<const int32_t *>(a.pe_idx)[e]);
            }
        } else if constexpr (BIAS == 1) {
            if (use[r]) {
                float *dst = bm + rowq_b + j;
                const int64_t e = (int64_t)b * a.bias_sb + (int64_t)nc * a.bias_sn + j;
                for (int h = 0; h < hn; ++h)
                    dst[h * PL] = load_any(a.bias, a.bias_dtype, e + (int64_t)(hb + h) * a.bias_sh) * LOG2E;
            }
        } else if constexpr (BIAS == 3) {
            if (use[r]) {
                float *dst = bm + rowq_b + j;
                const float2 g = *reinterpret_cast<const float2 *>(pos_b + (int64_t)idx[r] * a.pos_sn);
                for (int h = 0; h < hn; ++h)
                    dst[h * PL] = cont_bias(a.pos_w + (hb + h) * 5, a.pos_b[hb + h], g.x - pqx, g.y - pqy) * LOG2E;
            }
        } else {
            // no bias: zero entries, so that every (query, neighbour) pair still has its own code
            if (use[r])
                for (int h = 0; h < hn; ++h) bm[h * PL + rowq_b + j] = 0.f;
        }
    }
    auto table_row = [&](int r) -> int64_t {
        if constexpr (BIAS == 2) return prow[r];
        else return pe_from_coords32(pqx, pqy, gq[r].x, gq[r].y, float(a.rel_width), float(Tw));
    };
    // fp32 table, 4 heads: one 16-byte row per entry, loaded after the bits step and
    // stored to bm after the slots step
    float4 tv[RJ];
    float tsc[RJ];
    auto load_table_rows = [&]() {
        if constexpr (BIAS == 2 || BIAS == 4) {
            if (fast4) {
#pragma unroll
                for (int r = 0; r < RJ; ++r) {
                    tv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
                    tsc[r] = 0.f;
                    if (r >= nr || !use[r]) continue;
                    const int64_t row = table_row(r);
                    const bool in = row >= 0 && row < a.table_rows;
                    tsc[r] = in ? LOG2E : 0.f;
                    tv[r] = reinterpret_cast<const float4 *>(a.table)[((in ? row : 0) * H + hb) >> 2];
                }
            }
        }
    };
    auto write_table_biases = [&]() {
        if constexpr (BIAS == 2 || BIAS == 4) {
#pragma unroll
            for (int r = 0; r < RJ; ++r) {
                if (r >= nr || !use[r]) continue;
                float *dst = bm + rowq_b + (jl + LPQ * r);
                if (fast4) {
                    const float sc = tsc[r];
                    dst[0] = tv[r].x * sc;
                    dst[PL] = tv[r].y * sc;
                    dst[2 * PL] = tv[r].z * sc;
                    dst[3 * PL] = tv[r].w * sc;
                } else {
                    const int64_t row = table_row(r);
                    const bool in = row >= 0 && row < a.table_rows;
                    for (int h = 0; h < hn; ++h)
                        dst[h * PL] = in ? load_any(a.table, a.table_dtype, row * H + hb + h) * LOG2E : 0.f;
                }
            }
        }
    };
    // the cleared bits are visible before any wave sets one (the loads above stay
    // in flight across this barrier)
    lds_barrier();

    // ---- union: a flag byte (table modes) or bit per neighbour row of the index window
    // [wlo, wlo + 8192)
    const int wlo = max(0, min(n0 + TQ / 2 - WWORDS * 16, N - WWORDS * 32));
    bool outside = false;
#pragma unroll
    for (int r = 0; r < RJ; ++r) {
        if (r >= nr) continue;
        const unsigned o = unsigned(idx[r] - wlo);
        const bool in = o < unsigned(WWORDS * 32);
        outside = outside || (use[r] && !in);
        if (use[r] && in) {
            if constexpr (FLAGS) flg[o] = 1;  // every writer of a byte writes the same 1
            else atomicOr(&sh.s.bits[o >> 5], 1u << (o & 31));
        }
    }
    if (outside) red[0] = 1;
    {
        const float nm = grp8_sum(float(nmask));
        if (jl == 0) nmq_s[q] = nm;
    }
    lds_barrier();

    if constexpr (FLAGS) {
        // flags -> bits (thread t packs window word t); the -inf entries then take the
        // flags' place once every wave is past them
        const uint4 f0 = reinterpret_cast<const uint4 *>(flg)[2 * t];
        const uint4 f1 = reinterpret_cast<const uint4 *>(flg)[2 * t + 1];
        const uint32_t d[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        uint32_t wbits = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) wbits |= (((d[k] * 0x01020408u) >> 24) & 0xFu) << (4 * k);  // 4 flag bytes -> 4 bits
        sh.s.bits[t] = wbits;
        load_table_rows();
        lds_barrier();
        init_inf();
    } else {
        load_table_rows();
    }

    const bool flagged = (a.mask && a.mask_sh != 0) || red[0] != 0;
    if (!flagged && w == 0) {
        uint32_t c[4];
        int tot = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[i] = __popc(sh.s.bits[lane * 4 + i]);
            tot += c[i];
        }
        int inc = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(inc, o, 64);
            if (lane >= o) inc += v;
        }
        int ex = inc - tot;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sh.s.pref[lane * 4 + i] = ex;
            ex += c[i];
        }
        if (lane == 63) red[2] = inc;
    }
    lds_barrier();
    const int U = red[2];
    if (!PROJ && split && !flagged && U > UMAX) return true;
    // a half tile's 16 code rows take the 32 rows' space at twice the pitch: 2 UMAX slots
    const bool half = qhi - qlo == TQ / 2;
    const int pitch = half ? 2 * PWP : PWP;
    bool fallback = flagged || U > (half ? 2 * UMAX : UMAX);

    // ---- union slots; pw codes (plain stores: a code is unique to its (query, neighbour)
    // entry, so a repeated index within one query shows up as an overwritten code)
    int slot[RJ];
    if (!fallback) {
        const int rowq = (mine ? q - qlo : 0) * pitch;
#pragma unroll
        for (int r = 0; r < RJ; ++r) {
            slot[r] = 0;
            if (r >= nr) continue;
            const int o = min(max(idx[r] - wlo, 0), WWORDS * 32 - 1), wd = o >> 5, bt = o & 31;
            const int s_ = int(sh.s.pref[wd] + __popc(sh.s.bits[wd] & ((1u << bt) - 1u)));
            slot[r] = s_;
            if (use[r]) {
                ulist[s_] = idx[r];
                pw[rowq + s_] = uint8_t(jl + LPQ * r + 1);
            }
        }
        write_table_biases();
    }
    lds_barrier();
    if (!fallback) {
        bool dup = false;
        const int rowq = (mine ? q - qlo : 0) * pitch;
#pragma unroll
        for (int r = 0; r < RJ; ++r)
            if (r < nr && use[r])
                dup = dup || pw[rowq + slot[r]] != uint8_t(jl + LPQ * r + 1);
        if (__builtin_amdgcn_ballot_w64(dup) != 0 && lane == 0) red[1] = 1;
        lds_barrier();
        fallback = red[1] != 0;
    }

    if constexpr (!PROJ) {
        if (fallback) {
            tile_rows<T, BIAS>(a, b, n0 + qlo, qhi - qlo, hb, hn);
            return false;
        }
        // ---- head phase: wave w, heads hb + w, hb + w + NW, ... of the group
        wave_heads<T, BLANK>(a, b, n0, U, ulist, pw, bm, nmq_s[lane & 31], sh.vb[w], hb + w, NW, hb + hn, hb, HG, qlo,
                             qhi, pitch);
    } else {
        // every head of the image in this workgroup, at most one per wave (host-checked);
        // the [32][C] output block is staged in bm's space once every wave is past it
        const int C = H * HD, op = C + 8;
        uint16_t *otile = reinterpret_cast<uint16_t *>(bm);
        if (fallback) {
            // the per-row routine writes the tile's rows to out; they come back as the block
            tile_rows<T, BIAS>(a, b, n0, TQ, 0, H);
            __syncthreads();
            for (int e = t; e < TQ * (C / 8); e += THREADS) {
                const int qq = e / (C / 8), c8 = 8 * (e % (C / 8));
                uint4 v = make_uint4(0, 0, 0, 0);
                if (n0 + qq < N)
                    v = *reinterpret_cast<const uint4 *>(static_cast<const T *>(a.out) + (int64_t)b * a.o_sb +
                                                         (int64_t)(n0 + qq) * a.o_sn + c8);
                *reinterpret_cast<uint4 *>(otile + qq * op + c8) = v;
            }
            __syncthreads();
        } else {
            float yo[16];
            const bool has = w < H;
            if (has)
                wave_head_one<T, BLANK, true>(a, b, n0, U, ulist, pw, bm, nmq_s[lane & 31], sh.vb[w], w, 0, HG, yo);
            __syncthreads();
            if (has) {
                const int hh = lane >> 5, ql = lane & 31;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int c0 = w * HD + 8 * j + 4 * hh;
                    *reinterpret_cast<uint2 *>(otile + ql * op + c0) =
                        make_uint2(MM::pack2(yo[4 * j], yo[4 * j + 1]), MM::pack2(yo[4 * j + 2], yo[4 * j + 3]));
                }
            }
            __syncthreads();
        }
        proj_epilogue<T>(a, pj, b, n0, otile, op, C);
    }
    return false;
    };

    if (run(0, TQ, !PROJ)) {
        __syncthreads();  // every wave is past the full pass's LDS
        run(0, TQ / 2, false);
        __syncthreads();
        run(TQ / 2, TQ, false);
    }
}

using KernelFn = void (*)(const aff_nbhd_attn_args);

template <typename T, int D>
KernelFn pick_bias(int mode) {
    switch (mode) {
        case 0: return nbhd_attn_fwd_kernel<T, D, 0>;
        case 1: return nbhd_attn_fwd_kernel<T, D, 1>;
        case 2: return nbhd_attn_fwd_kernel<T, D, 2>;
        case 3: return nbhd_attn_fwd_kernel<T, D, 3>;
        default: return nbhd_attn_fwd_kernel<T, D, 4>;
    }
}

template <typename T>
KernelFn pick_d(int D, int mode) {
    switch (D) {
        case 8: return pick_bias<T, 8>(mode);
        case 16: return pick_bias<T, 16>(mode);
        case 32: return pick_bias<T, 32>(mode);
        case 64: return pick_bias<T, 64>(mode);
        case 128: return pick_bias<T, 128>(mode);
        default: return nullptr;
    }
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

inline int64_t tile_count(const aff_nbhd_attn_args &a) {
    return (int64_t)a.B * ((a.N + wt::TQ - 1) / wt::TQ);
}

// The wave-per-head kernel: 16-bit q/k/v, head_dim 32, M <= 64, every bias mode and
// head count, 32-bit offsets inside one image's q/k/v, index and mask planes.  One
// workgroup per (tile, head group) of wave_heads_per_group() heads: the group's
// per-(query, neighbour) bias store, TQ * (M + 1) * HG fp32 words, stays within
// MAXHM per query and the extra workgroups fill the chip when a stage has few tiles
// and many heads.
inline bool use_wave_path(const aff_nbhd_attn_args &a) {
    if (a.dtype == AFF_F32 || a.D != wt::HD || a.M > wt::MAXM) return false;
    // 32-bit byte offsets inside one (b, h) plane, built with 24-bit multiplies
    auto plane_ok = [&](int64_t sn) {
        return sn >= 0 && sn * 2 < ((int64_t)1 << 24) && ((int64_t)(a.N - 1) * sn + a.D) * 2 < ((int64_t)1 << 32);
    };
    if (!(a.N < (1 << 24) && plane_ok(a.q_sn) && plane_ok(a.k_sn) && plane_ok(a.v_sn))) return false;
    // set-up loads use 32-bit byte offsets inside one image's index and mask planes
    const int64_t lim = (int64_t)1 << 31;
    if (a.mi_sn < 0 || ((int64_t)a.N * a.mi_sn + a.M) * 8 >= lim) return false;
    if (a.mask && (a.mask_sn < 0 || (int64_t)a.N * a.mask_sn + a.M >= lim)) return false;
    return true;
}

// Heads per workgroup of the wave kernel: at most MAXHM / (M + 1) (the bias store) and MAXH.
inline int wave_heads_per_group(const aff_nbhd_attn_args &a) {
    int hg = wt::MAXHM / (a.M + 1);
    hg = hg < 1 ? 1 : (hg > wt::MAXH ? wt::MAXH : hg);
    return a.H < hg ? a.H : hg;
}

using WaveFn = void (*)(const aff_nbhd_attn_args, int, const ProjArgs);

template <typename T, int BIAS, bool PROJ>
WaveFn pick_wave3(bool i64, bool blank) {
    if (i64)
        return blank ? nbhd_attn_wave_kernel<T, BIAS, true, true, PROJ> : nbhd_attn_wave_kernel<T, BIAS, true, false, PROJ>;
    return blank ? nbhd_attn_wave_kernel<T, BIAS, false, true, PROJ> : nbhd_attn_wave_kernel<T, BIAS, false, false, PROJ>;
}

template <typename T, bool PROJ = false>
WaveFn pick_wave(const aff_nbhd_attn_args &a) {
    const bool i64 = a.idx_is_i64 != 0, blank = a.blank_k != nullptr;
    switch (a.bias_mode) {
        case 0: return pick_wave3<T, 0, PROJ>(i64, blank);
        case 1: return pick_wave3<T, 1, PROJ>(i64, blank);
        case 2: return pick_wave3<T, 2, PROJ>(i64, blank);
        case 3: return pick_wave3<T, 3, PROJ>(i64, blank);
        default: return pick_wave3<T, 4, PROJ>(i64, blank);
    }
}

}  // namespace attn
}  // namespace aff

using namespace aff;

extern "C" int aff_nbhd_attn_path(const aff_nbhd_attn_args *args) {
    if (args == nullptr) return -1;
    return attn::use_wave_path(*args) ? AFF_ATTN_PATH_WAVE : AFF_ATTN_PATH_ROW;
}

extern "C" size_t aff_nbhd_attn_workspace_bytes(const aff_nbhd_attn_args *args) {
    (void)args;
    return 0;
}

extern "C" aff_status aff_nbhd_attn_fwd(const aff_nbhd_attn_args *args, aff_stream_t stream) {
    AFF_CHECK_ARG(args != nullptr, "aff_nbhd_attn_fwd: NULL args");
    const aff_nbhd_attn_args &a = *args;
    AFF_CHECK_ARG(a.B >= 0 && a.H >= 1 && a.N >= 0 && a.M >= 0,
                  "aff_nbhd_attn_fwd: bad sizes B=%d H=%d N=%d M=%d", a.B, a.H, a.N, a.M);
    AFF_CHECK_ARG(a.D % 8 == 0 && a.D > 0, "aff_nbhd_attn_fwd: head_dim must be a multiple of 8 (D=%d)", a.D);
    if (a.D != 8 && a.D != 16 && a.D != 32 && a.D != 64 && a.D != 128)
        return fail(AFF_ERR_UNSUPPORTED, "aff_nbhd_attn_fwd: head_dim %d not compiled (8/16/32/64/128)", a.D);
    if (a.dtype != AFF_F32 && a.dtype != AFF_F16 && a.dtype != AFF_BF16)
        return fail(AFF_ERR_UNSUPPORTED, "aff_nbhd_attn_fwd: dtype %d", a.dtype);
    AFF_CHECK_ARG(a.bias_mode >= 0 && a.bias_mode <= 4, "aff_nbhd_attn_fwd: bias_mode %d", a.bias_mode);
    if ((int64_t)a.B * a.H * a.N == 0) return AFF_OK;
    AFF_CHECK_ARG(a.q && a.k && a.v && a.out, "aff_nbhd_attn_fwd: NULL q/k/v/out");
    AFF_CHECK_ARG(a.M == 0 || a.member_idx, "aff_nbhd_attn_fwd: NULL member_idx");
    AFF_CHECK_ARG((a.blank_k == nullptr) == (a.blank_v == nullptr),
                  "aff_nbhd_attn_fwd: blank_k and blank_v must both be set or both NULL");
    const int esz = a.dtype == AFF_F32 ? 4 : 2;
    // every 8-channel row piece must be 16-byte aligned for the vector loads
    const int64_t st[] = {a.q_sb, a.q_sh, a.q_sn, a.k_sb, a.k_sh, a.k_sn,
                          a.v_sb, a.v_sh, a.v_sn, a.o_sb, a.o_sh, a.o_sn};
    for (int64_t s : st) AFF_CHECK_ARG((s * esz) % 16 == 0, "aff_nbhd_attn_fwd: strides must keep 16-byte row alignment");
    AFF_CHECK_ARG(attn::aligned16(a.q) && attn::aligned16(a.k) && attn::aligned16(a.v) &&
                      attn::aligned16(a.out) && (!a.blank_k || (attn::aligned16(a.blank_k) && attn::aligned16(a.blank_v))),
                  "aff_nbhd_attn_fwd: q/k/v/out/blank pointers must be 16-byte aligned");
    if (a.bias_mode == 1) {
        AFF_CHECK_ARG(a.bias != nullptr, "aff_nbhd_attn_fwd: bias_mode 1 needs bias");
        AFF_CHECK_ARG(a.bias_dtype >= 0 && a.bias_dtype <= 2, "aff_nbhd_attn_fwd: bias dtype");
    } else if (a.bias_mode == 2) {
        AFF_CHECK_ARG(a.pe_idx && a.table, "aff_nbhd_attn_fwd: bias_mode 2 needs pe_idx and table");
        AFF_CHECK_ARG(a.table_dtype >= 0 && a.table_dtype <= 2, "aff_nbhd_attn_fwd: table dtype");
    } else if (a.bias_mode == 3) {
        AFF_CHECK_ARG(a.pos && a.pos_w && a.pos_b, "aff_nbhd_attn_fwd: bias_mode 3 needs pos, pos_w, pos_b");
    } else if (a.bias_mode == 4) {
        AFF_CHECK_ARG(a.pos && a.table, "aff_nbhd_attn_fwd: bias_mode 4 needs pos and table");
        AFF_CHECK_ARG(a.rel_width >= 1 && a.rel_width < 32768, "aff_nbhd_attn_fwd: rel_width %d", a.rel_width);
        AFF_CHECK_ARG(a.table_dtype >= 0 && a.table_dtype <= 2, "aff_nbhd_attn_fwd: table dtype");
    }
    hipStream_t hs = static_cast<hipStream_t>(stream);

    if (attn::use_wave_path(a)) {
        const int64_t ntiles = attn::tile_count(a);
        AFF_CHECK_ARG(ntiles < (int64_t)1 << 31, "aff_nbhd_attn_fwd: problem too large");
        const int hg = attn::wave_heads_per_group(a);
        const int64_t blocks = ntiles * ((a.H + hg - 1) / hg);
        AFF_CHECK_ARG(blocks < (int64_t)1 << 31, "aff_nbhd_attn_fwd: problem too large");
        const attn::WaveFn fn = a.dtype == AFF_BF16 ? attn::pick_wave<bf16_t>(a) : attn::pick_wave<f16_t>(a);
        hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(attn::THREADS), 0, hs, a, hg, attn::ProjArgs{nullptr, nullptr});
        return check_launch("aff_nbhd_attn_fwd (wave tiles)");
    }
    attn::KernelFn fn = nullptr;
    if (a.dtype == AFF_F32) fn = attn::pick_d<float>(a.D, a.bias_mode);
    else if (a.dtype == AFF_BF16) fn = attn::pick_d<bf16_t>(a.D, a.bias_mode);
    else fn = attn::pick_d<f16_t>(a.D, a.bias_mode);
    const int rows_per_block = attn::THREADS / (a.D / 8);
    const int64_t rows = (int64_t)a.B * a.H * a.N;
    const int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
    AFF_CHECK_ARG(blocks < (int64_t)1 << 31, "aff_nbhd_attn_fwd: problem too large");
    hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(attn::THREADS), 0, hs, a);
    return check_launch("aff_nbhd_attn_fwd");
}

extern "C" aff_status aff_nbhd_attn_proj_fwd(const aff_nbhd_attn_args *args, const void *proj_w, const float *proj_b,
                                             aff_stream_t stream) {
    AFF_CHECK_ARG(args != nullptr, "aff_nbhd_attn_proj_fwd: NULL args");
    const aff_nbhd_attn_args &a = *args;
    if (!(a.dtype == AFF_BF16 || a.dtype == AFF_F16) || a.D != attn::wt::HD || !attn::use_wave_path(a) ||
        a.H > attn::wt::NW || attn::wave_heads_per_group(a) < a.H)
        return fail(AFF_ERR_UNSUPPORTED,
                    "aff_nbhd_attn_proj_fwd: needs 16-bit q/k/v, head_dim 32, at most %d heads and M <= %d (H=%d M=%d D=%d)",
                    attn::wt::NW, attn::wt::MAXHM / (a.H > 0 ? a.H : 1) - 1, a.H, a.M, a.D);
    AFF_CHECK_ARG(proj_w && attn::aligned16(proj_w), "aff_nbhd_attn_proj_fwd: proj_w NULL or not 16-byte aligned");
    AFF_CHECK_ARG(a.o_sh == a.D && a.o_sn >= (int64_t)a.H * a.D,
                  "aff_nbhd_attn_proj_fwd: out must be [B, N, H * D] rows (o_sh = D)");
    AFF_CHECK_ARG(a.B >= 0 && a.N >= 0 && a.M >= 0, "aff_nbhd_attn_proj_fwd: bad sizes");
    if ((int64_t)a.B * a.N == 0) return AFF_OK;
    AFF_CHECK_ARG(a.q && a.k && a.v && a.out && (a.M == 0 || a.member_idx), "aff_nbhd_attn_proj_fwd: NULL pointer");
    AFF_CHECK_ARG((a.blank_k == nullptr) == (a.blank_v == nullptr), "aff_nbhd_attn_proj_fwd: blank_k / blank_v");
    const int64_t st16[] = {a.q_sb, a.q_sh, a.q_sn, a.k_sb, a.k_sh, a.k_sn, a.v_sb, a.v_sh, a.v_sn, a.o_sb, a.o_sn};
    for (int64_t s : st16) AFF_CHECK_ARG((s * 2) % 16 == 0, "aff_nbhd_attn_proj_fwd: strides must keep 16-byte rows");
    AFF_CHECK_ARG(attn::aligned16(a.q) && attn::aligned16(a.k) && attn::aligned16(a.v) && attn::aligned16(a.out),
                  "aff_nbhd_attn_proj_fwd: q/k/v/out must be 16-byte aligned");
    AFF_CHECK_ARG(a.bias_mode >= 0 && a.bias_mode <= 4, "aff_nbhd_attn_proj_fwd: bias_mode %d", a.bias_mode);
    if (a.bias_mode == 1) AFF_CHECK_ARG(a.bias, "aff_nbhd_attn_proj_fwd: bias_mode 1 needs bias");
    if (a.bias_mode == 2) AFF_CHECK_ARG(a.pe_idx && a.table, "aff_nbhd_attn_proj_fwd: bias_mode 2 needs pe_idx, table");
    if (a.bias_mode == 3) AFF_CHECK_ARG(a.pos && a.pos_w && a.pos_b, "aff_nbhd_attn_proj_fwd: bias_mode 3 inputs");
    if (a.bias_mode == 4)
        AFF_CHECK_ARG(a.pos && a.table && a.rel_width >= 1 && a.rel_width < 32768, "aff_nbhd_attn_proj_fwd: mode 4");
    const int64_t blocks = attn::tile_count(a);
    AFF_CHECK_ARG(blocks < (int64_t)1 << 31, "aff_nbhd_attn_proj_fwd: problem too large");
    const attn::WaveFn fn = a.dtype == AFF_BF16 ? attn::pick_wave<bf16_t, true>(a) : attn::pick_wave<f16_t, true>(a);
    hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(attn::THREADS), 0, static_cast<hipStream_t>(stream), a, a.H,
                       attn::ProjArgs{proj_w, proj_b});
    return check_launch("aff_nbhd_attn_proj_fwd");
}
