// Neighbourhood (cluster) flash attention, forward, for gfx950.
//
// Semantics: _nbhood_attn_fwd / _update_online_softmax_block in the
// reference (src/layers/kernels/local_attn.py:80-116, 119-215, 224-340):
// masked neighbours take the logit -1e11 and a zero value row, the per-head
// blank token joins the softmax after the neighbours, the running maximum
// starts at -1e11 and LSE = m + log(l + 1e-12).
//
// Layout: D/8 lanes own one (b, h, n) row; each lane holds 8 channels of q
// and of the accumulator.  Neighbours are consumed in blocks of 8: the 8
// index/mask/bias values and the 16 K/V row pieces are loaded before use so
// up to 16 gathers per lane are in flight, then one online-softmax rescale
// is applied per block.  Work is ordered (b, h, n) with n fastest and the
// block order is swizzled so each XCD walks a contiguous range: the K/V
// planes of one (b, h) (N * D * 4 bytes in bf16) stay resident in that XCD's
// L2 while its neighbour gathers run.
#include "common.hpp"

namespace aff {
namespace attn {

constexpr int THREADS = 256;
constexpr int NB = 8;  // neighbours per online-softmax block
constexpr float MASKED_LOGIT = -1e11f;

__device__ __forceinline__ int64_t load_index(const void *p, int is_i64, int64_t i) {
    return is_i64 ? static_cast<const int64_t *>(p)[i] : int64_t(static_cast<const int32_t *>(p)[i]);
}

// Table row of the relative offset (mx, my) - (qx, qy), evaluated with the
// encoder's fp32 operations in order (src/layers/aff.py:458-465):
//   rel = clamp(m - (q - W), 0, 2W);  pe = trunc(rel_y * (2W + 1) + rel_x)
__device__ __forceinline__ int64_t pe_from_coords(float qx, float qy, float mx, float my, float W,
                                                  float T) {
#pragma clang fp contract(off)
    float rx = mx - (qx - W), ry = my - (qy - W);
    rx = fminf(fmaxf(rx, 0.f), 2.f * W);
    ry = fminf(fmaxf(ry, 0.f), 2.f * W);
    return (int64_t)(ry * T + rx);
}

template <typename T, int D, int BIAS>
__global__ __launch_bounds__(THREADS) void nbhd_attn_fwd_kernel(const aff_nbhd_attn_args a) {
    using IO = ElemIO<T>;
    constexpr int LPR = D / 8;
    constexpr int ROWS = THREADS / LPR;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int sub = threadIdx.x % LPR;
    const int64_t row = (int64_t)bid * ROWS + threadIdx.x / LPR;
    const int64_t total = (int64_t)a.B * a.H * a.N;
    if (row >= total) return;  // whole lane groups leave together
    const int N = a.N, M = a.M, H = a.H;
    const int n = int(row % N);
    const int64_t bh = row / N;
    const int h = int(bh % H);
    const int b = int(bh / H);

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
                const float dx = mx - pqx, dy = my - pqy;
                const float r = sqrtf(dx * dx + dy * dy);
                const float sn = r > 0.f ? dy / r : 0.f, cs = r > 0.f ? dx / r : 0.f;
                bias[u] = pb + pw[0] * dx + pw[1] * dy + pw[2] * r + pw[3] * sn + pw[4] * cs;
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
    if (a.lse && sub == 0) a.lse[row] = lse;
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

}  // namespace attn
}  // namespace aff

using namespace aff;

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
