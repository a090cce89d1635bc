// Device helpers shared by the neighbourhood-attention forward (nbhd_attn.hip)
// and backward (nbhd_attn_bwd.hip) kernels.
#pragma once

#include "common.hpp"

namespace aff {
namespace attn {

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

// The same in 32-bit integers: every clamped offset gives a row below T * T.
__device__ __forceinline__ int pe_from_coords32(float qx, float qy, float mx, float my, float W, float T) {
#pragma clang fp contract(off)
    float rx = mx - (qx - W), ry = my - (qy - W);
    rx = fminf(fmaxf(rx, 0.f), 2.f * W);
    ry = fminf(fmaxf(ry, 0.f), 2.f * W);
    return int(ry * T + rx);
}

// Continuous relative-position features f(dx, dy) = (dx, dy, r, dy/r, dx/r).
__device__ __forceinline__ float cont_bias(const float *pw, float pb, float dx, float dy) {
    const float r = sqrtf(dx * dx + dy * dy);
    const float sn = r > 0.f ? dy / r : 0.f, cs = r > 0.f ? dx / r : 0.f;
    return pb + pw[0] * dx + pw[1] * dy + pw[2] * r + pw[3] * sn + pw[4] * cs;
}

}  // namespace attn
}  // namespace aff
