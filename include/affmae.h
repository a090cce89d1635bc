/*
 * affmae.h - C ABI of the MI355X (gfx950) point-token hot path.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * launches on the caller's HIP stream and returns without synchronising.
 * The library never allocates or frees device memory: outputs and workspace
 * are owned by the caller.  Errors are returned as aff_status codes, with a
 * thread-local message available from aff_last_error().
 *
 * Reference interfaces replaced (paths relative to the najafian-lab/affmae
 * tree; that project launches Triton kernels from Python and has no FFI of
 * its own, so each entry point replaces the Python launcher named beside it).
 */
#ifndef AFFMAE_H
#define AFFMAE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A hipStream_t handle; NULL selects the null stream. */
typedef void *aff_stream_t;

typedef enum aff_status {
    AFF_OK = 0,
    AFF_ERR_INVALID_ARG = 1, /* shape / stride / pointer contract violated   */
    AFF_ERR_UNSUPPORTED = 2, /* valid request outside the compiled variants   */
    AFF_ERR_WORKSPACE = 3,   /* workspace pointer NULL or smaller than needed */
    AFF_ERR_LAUNCH = 4       /* the HIP runtime rejected a kernel launch      */
} aff_status;

typedef enum aff_dtype { AFF_F32 = 0, AFF_F16 = 1, AFF_BF16 = 2 } aff_dtype;

/* Message describing the last non-AFF_OK status returned on this thread. */
const char *aff_last_error(void);

/* Incremented whenever a struct layout or signature below changes. */
int aff_abi_version(void);

/* ------------------------------------------------------------------------ *
 * Exact K-nearest-neighbour search over 2-D points.
 *
 * Replaces: knn_forward()  src/layers/kernels/knn.py:1368-1540
 *           (and its k>8 fallback knn_large_k_fallback() knn.py:1335-1365)
 *
 * query[b, m, 0:2], ref[b, n, 0:2] are fp32; the coordinate stride is 1,
 * q_sb/q_sm and r_sb/r_sn are element strides of the batch and point dims.
 * For every query the k reference points with the smallest key
 *     (d2, n),  d2 = fl(fl(dx*dx) + fl(dy*dy)),  dx = fl(qx - rx), dy = fl(qy - ry)
 * are written in ascending key order, i.e. by distance and, on equal
 * distance, by lower reference index.  Requires 1 <= k <= N, N >= 1 and
 * finite coordinates.  out_idx is [B, M, k] contiguous, int32 or int64
 * (idx_is_i64 != 0).  out_d2 ([B, M, k] fp32) may be NULL.
 * ws must hold aff_knn_workspace_bytes(B, M, N, D, k) bytes.
 * Only D == 2 is implemented; other D return AFF_ERR_UNSUPPORTED.
 * ------------------------------------------------------------------------ */
size_t aff_knn_workspace_bytes(int B, int M, int N, int D, int k);

aff_status aff_knn(const float *query, int64_t q_sb, int64_t q_sm,
                   const float *ref, int64_t r_sb, int64_t r_sn,
                   int B, int M, int N, int D, int k,
                   void *out_idx, int idx_is_i64, float *out_d2,
                   void *ws, size_t ws_bytes, aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Neighbourhood (cluster) flash attention, forward.
 *
 * Replaces: launch_flash_nbhood_attn_fwd()  src/layers/kernels/local_attn.py:609-708
 *           kernel semantics _nbhood_attn_fwd  local_attn.py:224-340
 *
 * For each (b, h, n):
 *   s_j = valid_j ? scale * <q, k[idx_j]> + bias_j : -1e11      (j < M)
 *   s_blank = scale * <q, blank_k[h]>                           (if blank)
 *   m = max(-1e11, s_*),  l = sum exp(s_* - m)
 *   lse = m + log(l + 1e-12),  out = exp(m - lse) * sum p_* v_*
 * where valid_j = mask[b,h,n,j] != 0 (all valid without a mask) and
 * 0 <= idx_j < N (an out-of-range index is treated as masked), and
 * masked neighbours contribute a zero value row.
 *
 * q/k/v/out: dtype `dtype`, logical [B, H, N, D] with element strides
 * (sb, sh, sn) and a unit stride on D.  D must be 8, 16, 32, 64 or 128.
 * member_idx: [B, N, M] int32 or int64, unit stride on M.
 * bias_mode:
 *   0  no bias
 *   1  dense bias[B, H, N, M] (bias_dtype), unit stride on M
 *   2  table: bias = table[pe_idx[b, n, j], h]; table is [table_rows, H]
 *      contiguous (table_dtype), pe_idx [B, N, M] int32/int64, unit stride
 *      on M; rows outside [0, table_rows) read as 0
 *   3  continuous: bias = pos_w[h, :] . f(p[idx_j] - p[n]) + pos_b[h] with
 *      f(dx, dy) = (dx, dy, r, dy / r, dx / r), r = sqrt(dx^2 + dy^2),
 *      and the last two features 0 when r == 0; pos is [B, N, 2] fp32.
 *   4  table indexed from coordinates: bias = table[pe, h] with pe computed
 *      in-kernel exactly as the encoder builds pe_idx
 *      (src/layers/aff.py:458-465, fp32, no contraction):
 *        rel = clamp(p[idx_j] - (p[n] - W), 0, 2W),  W = rel_width,
 *        pe  = trunc(rel.y * (2W + 1) + rel.x)
 *      pos is [B, N, 2] fp32, table as in mode 2 (table_rows = (2W+1)^2).
 * mask: uint8 [B, H, N, M] with strides (mask_sb, mask_sh, mask_sn), unit
 *       stride on M; mask_sh == 0 broadcasts one mask over heads. NULL = none.
 * blank_k/blank_v: [H, D] contiguous in `dtype`, both NULL or both set.
 * lse: [B, H, N] fp32 contiguous, may be NULL.
 * ------------------------------------------------------------------------ */
typedef struct aff_nbhd_attn_args {
    int dtype; /* aff_dtype of q, k, v, out, blank_k, blank_v */
    int B, H, N, M, D;
    float scale;
    const void *q; int64_t q_sb, q_sh, q_sn;
    const void *k; int64_t k_sb, k_sh, k_sn;
    const void *v; int64_t v_sb, v_sh, v_sn;
    const void *member_idx; int idx_is_i64; int64_t mi_sb, mi_sn;
    int bias_mode;
    const void *bias; int bias_dtype; int64_t bias_sb, bias_sh, bias_sn;
    const void *pe_idx; int pe_is_i64; int64_t pe_sb, pe_sn;
    const void *table; int table_dtype; int64_t table_rows;
    const float *pos; int64_t pos_sb, pos_sn;
    int rel_width;      /* W of bias mode 4 (127 in the reference) */
    const float *pos_w; /* [H, 5] */
    const float *pos_b; /* [H]    */
    const uint8_t *mask; int64_t mask_sb, mask_sh, mask_sn;
    const void *blank_k;
    const void *blank_v;
    void *out; int64_t o_sb, o_sh, o_sn;
    float *lse;
} aff_nbhd_attn_args;

aff_status aff_nbhd_attn_fwd(const aff_nbhd_attn_args *args, aff_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* AFFMAE_H */
