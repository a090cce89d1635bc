// Neighbourhood index construction of the encoder's BasicLayer for gfx950:
// the member gather, the padding-mask gather and the relative-position table
// index, fused into one pass (reference src/layers/aff.py:452-465).
//
// For every token n of image b and every slot j < nnc * m of its
// neighbourhood, with c = nearest[b, n, j / m] (the j / m-th nearest
// cluster) and i = j % m:
//   member[b, n, j] = members[b, c, i]
//   mask[b, n, j]   = cmask[b, c, i] != 0                   (when cmask is given)
//   pe[b, n, j]     = trunc(rel_y * (2W + 1) + rel_x),  rel = clamp(pos[member] - (pos[n] - W), 0, 2W)
// in fp32 with no contraction, exactly the reference's tensor expression
// (each product and sum rounded on its own).  A cluster id outside [0, K) or a
// member outside [0, N) gives member 0, mask 0 and pe of member 0.
//
// One lane per output element; the lanes of a token read its nearest-cluster
// row and its own coordinates once per 64 slots through the L1, the cluster
// member rows and member coordinates are gathers.  Bandwidth-bound: the three
// outputs are the only large traffic.
#include "common.hpp"

namespace aff {
namespace nidx {

constexpr int THREADS = 256;

struct Args {
    const void *nearest; int near_i64; int64_t n_sb, n_sn;
    const void *members; int mem_i64; int64_t m_sb, m_sk;
    const uint8_t *cmask; int64_t c_sb, c_sk;
    const float *pos; int64_t p_sb, p_sn;
    int B, N, K, nnc, m, rel_width;
    void *out_member; int out_i64;
    uint8_t *out_mask;
    void *out_pe; int pe_i64;
};

__device__ __forceinline__ int64_t ld_index(const void *p, int i64, int64_t e) {
    return i64 ? static_cast<const int64_t *>(p)[e] : int64_t(static_cast<const int32_t *>(p)[e]);
}

__device__ __forceinline__ int64_t pe_index(float qx, float qy, float mx, float my, float W, float T) {
#pragma clang fp contract(off)
    float rx = mx - (qx - W), ry = my - (qy - W);
    rx = fminf(fmaxf(rx, 0.f), 2.f * W);
    ry = fminf(fmaxf(ry, 0.f), 2.f * W);
    const float ty = ry * T;
    return (int64_t)(ty + rx);
}

__global__ __launch_bounds__(THREADS) void cluster_members_kernel(const Args a) {
    const int S = a.nnc * a.m;
    const int64_t e = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * THREADS + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.N * S;
    if (e >= total) return;
    const int j = int(e % S);
    const int64_t bn = e / S;
    const int n = int(bn % a.N), b = int(bn / a.N);
    const int ci = j / a.m, i = j - ci * a.m;
    const int64_t c = ld_index(a.nearest, a.near_i64, (int64_t)b * a.n_sb + (int64_t)n * a.n_sn + ci);
    const bool cok = c >= 0 && c < a.K;
    int64_t mem = 0;
    bool keep = false;
    if (cok) {
        mem = ld_index(a.members, a.mem_i64, (int64_t)b * a.m_sb + c * a.m_sk + i);
        keep = a.cmask ? a.cmask[(int64_t)b * a.c_sb + c * a.c_sk + i] != 0 : true;
        if (mem < 0 || mem >= a.N) {
            mem = 0;
            keep = false;
        }
    }
    if (a.out_i64) static_cast<int64_t *>(a.out_member)[e] = mem;
    else static_cast<int32_t *>(a.out_member)[e] = int32_t(mem);
    if (a.out_mask) a.out_mask[e] = keep ? 1 : 0;
    if (a.out_pe) {
        const float *pb = a.pos + (int64_t)b * a.p_sb;
        const float2 q = make_float2(pb[(int64_t)n * a.p_sn], pb[(int64_t)n * a.p_sn + 1]);
        const float2 p = make_float2(pb[mem * a.p_sn], pb[mem * a.p_sn + 1]);
        const float W = float(a.rel_width), T = float(2 * a.rel_width + 1);
        const int64_t pe = pe_index(q.x, q.y, p.x, p.y, W, T);
        if (a.pe_i64) static_cast<int64_t *>(a.out_pe)[e] = pe;
        else static_cast<int32_t *>(a.out_pe)[e] = int32_t(pe);
    }
}

}  // namespace nidx
}  // namespace aff

using namespace aff;

extern "C" aff_status aff_cluster_members(const void *nearest, int near_is_i64, int64_t n_sb, int64_t n_sn,
                                          const void *members, int mem_is_i64, int64_t m_sb, int64_t m_sk,
                                          const uint8_t *cmask, int64_t c_sb, int64_t c_sk,
                                          const float *pos, int64_t p_sb, int64_t p_sn,
                                          int B, int N, int K, int nnc, int m, int rel_width,
                                          void *out_member, int out_is_i64, uint8_t *out_mask,
                                          void *out_pe, int pe_is_i64, aff_stream_t stream) {
    AFF_CHECK_ARG(B >= 0 && N >= 0 && K >= 1 && nnc >= 0 && m >= 1,
                  "aff_cluster_members: bad sizes B=%d N=%d K=%d nnc=%d m=%d", B, N, K, nnc, m);
    AFF_CHECK_ARG(nnc <= K, "aff_cluster_members: nnc=%d exceeds the number of clusters K=%d", nnc, K);
    const int64_t total = (int64_t)B * N * nnc * m;
    if (total == 0) return AFF_OK;
    AFF_CHECK_ARG(nearest && members && out_member, "aff_cluster_members: NULL nearest/members/out_member");
    AFF_CHECK_ARG(!out_pe || pos, "aff_cluster_members: pe output needs pos");
    AFF_CHECK_ARG(!out_pe || (rel_width >= 1 && rel_width < 32768), "aff_cluster_members: rel_width %d", rel_width);
    const int64_t blocks = (total + nidx::THREADS - 1) / nidx::THREADS;
    AFF_CHECK_ARG(blocks < (int64_t)1 << 31, "aff_cluster_members: problem too large");
    const nidx::Args a{nearest, near_is_i64, n_sb, n_sn, members, mem_is_i64, m_sb, m_sk, cmask, c_sb, c_sk,
                       pos, p_sb, p_sn, B, N, K, nnc, m, rel_width, out_member, out_is_i64, out_mask,
                       out_pe, pe_is_i64};
    hipLaunchKernelGGL(nidx::cluster_members_kernel, dim3((unsigned)blocks), dim3(nidx::THREADS), 0,
                       static_cast<hipStream_t>(stream), a);
    return check_launch("aff_cluster_members");
}
