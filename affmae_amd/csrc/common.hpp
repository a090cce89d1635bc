// Shared device/host helpers for the gfx950 kernels behind include/affmae.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "affmae.h"

namespace aff {

// ---------------------------------------------------------------- errors --
// Thread-local message for aff_last_error(); set by fail().
aff_status fail(aff_status code, const char *fmt, ...);
void clear_error();

#define AFF_CHECK_ARG(cond, ...)                                   \
    do {                                                           \
        if (!(cond)) return ::aff::fail(AFF_ERR_INVALID_ARG, __VA_ARGS__); \
    } while (0)

// Compute units of the current device (cached per device id; 0 -> 256).
int device_cu_count();

inline aff_status check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(AFF_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return AFF_OK;
}

// -------------------------------------------------------- number formats --
struct bf16_t { uint16_t bits; };
struct f16_t { _Float16 v; };

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(uint32_t(b) << 16);
}
// Round to nearest even (gfx950's v_cvt_pk_bf16_f32); NaN stays a NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Element-type traits: storage type, vector load of 8 elements into fp32.
template <typename T> struct ElemIO;

template <> struct ElemIO<float> {
    using storage = float;
    static constexpr aff_dtype code = AFF_F32;
    __device__ __forceinline__ static void load8(const float *p, float (&o)[8]) {
        const float4 *v = reinterpret_cast<const float4 *>(p);
        float4 a = v[0], b = v[1];
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    }
    __device__ __forceinline__ static void store8(float *p, const float (&o)[8]) {
        float4 *v = reinterpret_cast<float4 *>(p);
        v[0] = make_float4(o[0], o[1], o[2], o[3]);
        v[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
    __device__ __forceinline__ static float load1(const float *p) { return *p; }
    struct raw8 { float4 a, b; };
    __device__ __forceinline__ static raw8 load_raw(const float *p) {
        const float4 *v = reinterpret_cast<const float4 *>(p);
        return raw8{v[0], v[1]};
    }
    __device__ __forceinline__ static void cvt(const raw8 &r, float (&o)[8]) {
        o[0] = r.a.x; o[1] = r.a.y; o[2] = r.a.z; o[3] = r.a.w;
        o[4] = r.b.x; o[5] = r.b.y; o[6] = r.b.z; o[7] = r.b.w;
    }
};

template <> struct ElemIO<bf16_t> {
    using storage = bf16_t;
    static constexpr aff_dtype code = AFF_BF16;
    __device__ __forceinline__ static void load8(const bf16_t *p, float (&o)[8]) {
        uint4 u = *reinterpret_cast<const uint4 *>(p);
        uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __uint_as_float(w[i] << 16);
            o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
    __device__ __forceinline__ static void store8(bf16_t *p, const float (&o)[8]) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = uint32_t(f32_to_bf16(o[2 * i])) | (uint32_t(f32_to_bf16(o[2 * i + 1])) << 16);
        *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    __device__ __forceinline__ static float load1(const bf16_t *p) { return bf16_to_f32(p->bits); }
    using raw8 = uint4;
    __device__ __forceinline__ static raw8 load_raw(const bf16_t *p) {
        return *reinterpret_cast<const uint4 *>(p);
    }
    __device__ __forceinline__ static void cvt(const raw8 &u, float (&o)[8]) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __uint_as_float(w[i] << 16);
            o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
};

template <> struct ElemIO<f16_t> {
    using storage = f16_t;
    static constexpr aff_dtype code = AFF_F16;
    __device__ __forceinline__ static void load8(const f16_t *p, float (&o)[8]) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 v = *reinterpret_cast<const h8 *>(p);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = float(v[i]);
    }
    __device__ __forceinline__ static void store8(f16_t *p, const float (&o)[8]) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = _Float16(o[i]);
        *reinterpret_cast<h8 *>(p) = v;
    }
    __device__ __forceinline__ static float load1(const f16_t *p) { return float(p->v); }
    using raw8 = uint4;
    __device__ __forceinline__ static raw8 load_raw(const f16_t *p) {
        return *reinterpret_cast<const uint4 *>(p);
    }
    __device__ __forceinline__ static void cvt(const raw8 &u, float (&o)[8]) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 v = __builtin_bit_cast(h8, u);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = float(v[i]);
    }
};

// Scalar load of any supported dtype selected at run time (cold paths only).
__device__ __forceinline__ float load_any(const void *p, int dtype, int64_t i) {
    if (dtype == AFF_F32) return static_cast<const float *>(p)[i];
    if (dtype == AFF_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    return float(static_cast<const _Float16 *>(p)[i]);
}

// ---------------------------------------------------------- cross-lane ----
// XOR butterfly within a wave64.  Masks 1 and 2 use DPP quad permutes; the
// rest go through ds_swizzle / bpermute via __shfl_xor.
template <int MASK>
__device__ __forceinline__ float xor_lane(float v) {
    if constexpr (MASK == 1) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
    } else if constexpr (MASK == 2) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
    } else {
        return __shfl_xor(v, MASK, 64);
    }
}

// Data-parallel-primitive move with a compile-time control word.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Max / sum over each aligned row of 16 lanes, result in every lane of the
// row: two quad butterflies (quad_perm [1,0,3,2] and [2,3,0,1]) leave each
// lane with its quad's value, then row rotations by 4 and 8 fold in the other
// three quads.  All DPP, no LDS-unit permutes.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x124>(v));
    return fmaxf(v, dpp_mov<0x128>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x124>(v);
    return v + dpp_mov<0x128>(v);
}

// Sum over aligned groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += xor_lane<1>(v);
    if constexpr (G >= 4) v += xor_lane<2>(v);
    if constexpr (G >= 8) v += xor_lane<4>(v);
    if constexpr (G >= 16) v += xor_lane<8>(v);
    if constexpr (G >= 32) v += xor_lane<16>(v);
    if constexpr (G >= 64) v += xor_lane<32>(v);
    return v;
}

// Workgroup barrier for kernels whose threads communicate only through LDS:
// waits for this wave's LDS operations, not for its global loads (which
// __syncthreads() also drains), so prefetched global data stays in flight
// across the barrier.  Global results read by other threads need __syncthreads().
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Map a linear block id so that consecutive work items stay on one XCD.
// Hardware dispatches block i to XCD (i % 8); this returns the position of
// block i in an order where XCD x owns the contiguous range
// [x * per, (x + 1) * per) of the work list.
__device__ __forceinline__ uint32_t xcd_swizzle(uint32_t bid, uint32_t nblocks) {
    constexpr uint32_t NXCD = 8;
    uint32_t per = nblocks / NXCD;          // full rounds
    uint32_t rem = nblocks % NXCD;
    uint32_t xcd = bid % NXCD, slot = bid / NXCD;
    if (slot >= per) return per * NXCD + xcd;  // tail blocks: leave in place
    (void)rem;
    return xcd * per + slot;
}

}  // namespace aff
