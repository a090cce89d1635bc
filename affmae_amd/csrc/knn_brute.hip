// Exact K-nearest-neighbour search over 3-D and 4-D points for gfx950
// (aff_knn with D != 2; reference src/layers/kernels/knn.py:340-419, 474-581
// for the D = 3 / 4 kernels, :1312-1365 for k > 8).
//
// Same contract as the 2-D search: for each query the k reference points of
// smallest key (d2, n), d2 = sum over the dimensions in order of fl(diff^2)
// (no contraction), ascending.  One lane per query keeps its best KT keys
// (64-bit: the d2 bits over the index) sorted in registers (in LDS for
// k > 16); the workgroup
// streams the reference points through LDS in tiles of TILE points.  Every
// lane reads the same LDS word at a time (a broadcast), so the loop is bound
// by the VALU distance and compare work (D + 2 ops per pair when no insert).
#include "common.hpp"
#include "knn_brute.hpp"

namespace aff {
namespace knnb {

constexpr int THREADS = 256;
constexpr int TILE = 1024;

template <int D, int KT>
__global__ __launch_bounds__(THREADS) void knn_brute_kernel(const float *query, int64_t q_sb, int64_t q_sm,
                                                            const float *ref, int64_t r_sb, int64_t r_sn, int M,
                                                            int N, int k, void *out_idx, int idx_i64, float *out_d2) {
    __shared__ float4 tile[TILE];
    const int b = blockIdx.y;
    const int m = blockIdx.x * THREADS + threadIdx.x;
    const bool act = m < M;
    float q[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) {
#pragma unroll
        for (int d = 0; d < D; ++d) q[d] = query[(int64_t)b * q_sb + (int64_t)m * q_sm + d];
    }
    uint64_t keys[KT];
#pragma unroll
    for (int i = 0; i < KT; ++i) keys[i] = ~uint64_t(0);
    const float *R = ref + (int64_t)b * r_sb;
    for (int t0 = 0; t0 < N; t0 += TILE) {
        const int tn = min(TILE, N - t0);
        __syncthreads();
        for (int i = threadIdx.x; i < tn; i += THREADS) {
            const float *p = R + (int64_t)(t0 + i) * r_sn;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            v.x = p[0];
            if (D > 1) v.y = p[1];
            if (D > 2) v.z = p[2];
            if (D > 3) v.w = p[3];
            tile[i] = v;
        }
        __syncthreads();
        for (int i = 0; i < tn; ++i) {
            const float4 p = tile[i];
            const float pc[4] = {p.x, p.y, p.z, p.w};
            float d2 = 0.f;
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const float df = q[d] - pc[d];
                float sq = df * df;
                asm volatile("" : "+v"(sq));  // keep the square rounded on its own
                d2 = d == 0 ? sq : d2 + sq;
            }
            const uint64_t key = (uint64_t(__float_as_uint(d2)) << 32) | uint32_t(t0 + i);
            if (key < keys[KT - 1]) {
#pragma unroll
                for (int j = KT - 1; j > 0; --j) {
                    const uint64_t prev = keys[j - 1];
                    keys[j] = key < prev ? prev : (key < keys[j] ? key : keys[j]);
                }
                keys[0] = key < keys[0] ? key : keys[0];
            }
        }
    }
    if (!act) return;
    const int64_t o = ((int64_t)b * M + m) * k;
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        if (j >= k) break;
        const int n = int(uint32_t(keys[j]));
        if (idx_i64) static_cast<int64_t *>(out_idx)[o + j] = n;
        else static_cast<int32_t *>(out_idx)[o + j] = n;
        if (out_d2) out_d2[o + j] = __uint_as_float(uint32_t(keys[j] >> 32));
    }
}

// k > 16: each lane's sorted list lives in LDS (one wave per workgroup, the
// list of lane l in column l so that the 64 lanes hit 64 distinct banks),
// the current worst key in a register.
template <int D, int KT>
__global__ __launch_bounds__(64) void knn_brute_lds_kernel(const float *query, int64_t q_sb, int64_t q_sm,
                                                           const float *ref, int64_t r_sb, int64_t r_sn, int M,
                                                           int N, int k, void *out_idx, int idx_i64, float *out_d2) {
    constexpr int LT = 1024;
    __shared__ float4 tile[LT];
    __shared__ uint64_t list[KT][64];
    const int lane = threadIdx.x;
    const int b = blockIdx.y;
    const int m = blockIdx.x * 64 + lane;
    const bool act = m < M;
    float q[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) {
#pragma unroll
        for (int d = 0; d < D; ++d) q[d] = query[(int64_t)b * q_sb + (int64_t)m * q_sm + d];
    }
    for (int j = 0; j < KT; ++j) list[j][lane] = ~uint64_t(0);
    uint64_t worst = ~uint64_t(0);
    const float *R = ref + (int64_t)b * r_sb;
    for (int t0 = 0; t0 < N; t0 += LT) {
        const int tn = min(LT, N - t0);
        __syncthreads();
        for (int i = lane; i < tn; i += 64) {
            const float *p = R + (int64_t)(t0 + i) * r_sn;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            v.x = p[0];
            if (D > 1) v.y = p[1];
            if (D > 2) v.z = p[2];
            if (D > 3) v.w = p[3];
            tile[i] = v;
        }
        __syncthreads();
        for (int i = 0; i < tn; ++i) {
            const float4 p = tile[i];
            const float pc[4] = {p.x, p.y, p.z, p.w};
            float d2 = 0.f;
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const float df = q[d] - pc[d];
                float sq = df * df;
                asm volatile("" : "+v"(sq));
                d2 = d == 0 ? sq : d2 + sq;
            }
            const uint64_t key = (uint64_t(__float_as_uint(d2)) << 32) | uint32_t(t0 + i);
            if (key < worst) {
                int j = KT - 1;
                while (j > 0) {
                    const uint64_t prev = list[j - 1][lane];
                    if (prev <= key) break;
                    list[j][lane] = prev;
                    --j;
                }
                list[j][lane] = key;
                worst = list[KT - 1][lane];
            }
        }
    }
    if (!act) return;
    const int64_t o = ((int64_t)b * M + m) * k;
    for (int j = 0; j < k; ++j) {
        const uint64_t key = list[j][lane];
        const int n = int(uint32_t(key));
        if (idx_i64) static_cast<int64_t *>(out_idx)[o + j] = n;
        else static_cast<int32_t *>(out_idx)[o + j] = n;
        if (out_d2) out_d2[o + j] = __uint_as_float(uint32_t(key >> 32));
    }
}

using Fn = void (*)(const float *, int64_t, int64_t, const float *, int64_t, int64_t, int, int, int, void *, int,
                    float *);

template <int D>
Fn pick_k(int k) {
    if (k <= 4) return knn_brute_kernel<D, 4>;
    if (k <= 8) return knn_brute_kernel<D, 8>;
    if (k <= 16) return knn_brute_kernel<D, 16>;
    if (k <= 32) return knn_brute_lds_kernel<D, 32>;
    return knn_brute_lds_kernel<D, 64>;
}

}  // namespace knnb

aff_status knn_brute_launch(const float *query, int64_t q_sb, int64_t q_sm, const float *ref, int64_t r_sb,
                            int64_t r_sn, int B, int M, int N, int D, int k, void *out_idx, int idx_is_i64,
                            float *out_d2, hipStream_t stream) {
    if (k > KNN_BRUTE_KMAX)
        return fail(AFF_ERR_UNSUPPORTED, "aff_knn: D=%d supports k <= %d (got k=%d)", D, KNN_BRUTE_KMAX, k);
    AFF_CHECK_ARG(B <= 65535, "aff_knn: B=%d exceeds 65535", B);
    knnb::Fn fn = D == 1 ? knnb::pick_k<1>(k) : D == 3 ? knnb::pick_k<3>(k) : knnb::pick_k<4>(k);
    const int threads = k <= 16 ? knnb::THREADS : 64;
    dim3 grid((M + threads - 1) / threads, B);
    hipLaunchKernelGGL(fn, grid, dim3(threads), 0, stream, query, q_sb, q_sm, ref, r_sb, r_sn, M, N, k, out_idx,
                       idx_is_i64, out_d2);
    return check_launch("aff_knn (brute force)");
}

}  // namespace aff
