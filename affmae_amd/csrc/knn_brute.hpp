// Exact K-NN over D = 1, 3 or 4 dimensional points (knn_brute.hip); aff_knn
// calls it for every D other than 2.
#pragma once

#include "common.hpp"

namespace aff {

constexpr int KNN_BRUTE_KMAX = 64;

aff_status knn_brute_launch(const float *query, int64_t q_sb, int64_t q_sm, const float *ref, int64_t r_sb,
                            int64_t r_sn, int B, int M, int N, int D, int k, void *out_idx, int idx_is_i64,
                            float *out_d2, hipStream_t stream);

}  // namespace aff
