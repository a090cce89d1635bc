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
 * Exact K-nearest-neighbour search over 2-D (and 1-, 3-, 4-D) points.
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
 * D == 2 runs the grid-bucketed search (any k).  D == 1, 3 or 4 (the
 * reference's D = 3 / 4 kernels, knn.py:340-419, 474-581) runs an exact
 * brute-force search with k <= 64 and no workspace; query / ref then hold D
 * coordinates per point (unit stride) and the sum of squares runs over the
 * dimensions in order.  Other D, or k > 64 with D != 2, return
 * AFF_ERR_UNSUPPORTED.
 * ------------------------------------------------------------------------ */
size_t aff_knn_workspace_bytes(int B, int M, int N, int D, int k);

aff_status aff_knn(const float *query, int64_t q_sb, int64_t q_sm,
                   const float *ref, int64_t r_sb, int64_t r_sn,
                   int B, int M, int N, int D, int k,
                   void *out_idx, int idx_is_i64, float *out_d2,
                   void *ws, size_t ws_bytes, aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * aff_knn without a caller workspace.
 *
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same search and outputs as aff_knn, with the
 * workspace taken from a static device array of AFF_KNN_NOALLOC_SCRATCH_BYTES
 * that each GPU the library runs on holds until the process ends.  Calls
 * needing more than that (aff_knn_workspace_bytes) fail with
 * AFF_ERR_WORKSPACE.  Allocates nothing.  All calls on one GPU share its
 * array: calls that overlap on one GPU (several streams or host threads) race
 * and must be serialised by the caller.
 * ------------------------------------------------------------------------ */
#define AFF_KNN_NOALLOC_SCRATCH_BYTES (16u << 20)

aff_status aff_knn_noalloc(const float *query, int64_t q_sb, int64_t q_sm,
                           const float *ref, int64_t r_sb, int64_t r_sn,
                           int B, int M, int N, int D, int k,
                           void *out_idx, int idx_is_i64, float *out_d2,
                           aff_stream_t stream);

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
    void *ws; size_t ws_bytes; /* workspace: aff_nbhd_attn_workspace_bytes(args) bytes (0 today) */
} aff_nbhd_attn_args;

/* Workspace the call with these arguments needs: 0 (the kernels keep every
 * per-tile table in LDS); kept so callers can size args->ws generically. */
size_t aff_nbhd_attn_workspace_bytes(const aff_nbhd_attn_args *args);
aff_status aff_nbhd_attn_fwd(const aff_nbhd_attn_args *args, aff_stream_t stream);

/* Which kernel family aff_nbhd_attn_fwd would run for these arguments (no
 * launch, no validation beyond the path predicates).  A diagnostic with no
 * counterpart in the reference: tests use it to show which path a case takes.
 *   AFF_ATTN_PATH_ROW   per-row kernel (any dtype / head_dim)
 *   AFF_ATTN_PATH_WAVE  16-bit MFMA kernel: 32-query tiles, one wave per head,
 *                       workgroups of up to 4 heads (head_dim 32, M <= 64)
 * Returns -1 for a NULL pointer. */
enum { AFF_ATTN_PATH_ROW = 0, AFF_ATTN_PATH_WAVE = 2 };
int aff_nbhd_attn_path(const aff_nbhd_attn_args *args);


/* ------------------------------------------------------------------------ *
 * Neighbourhood attention with ClusterAttention's output projection fused.
 *
 * Replaces: the attention (as aff_nbhd_attn_fwd) followed by
 *           out = self.proj(out)   src/layers/attention.py:204-205
 *
 * args as for aff_nbhd_attn_fwd, except that args->out receives the
 * projected rows y[b, n, :] = O[b, n, :] proj_w^T + proj_b, with O[b, n, :]
 * the attention output of all heads concatenated ([B, N, H * D], o_sh = D,
 * o_sn >= H * D).  proj_w: [H*D, H*D] in the attention dtype, row o = output
 * channel o (nn.Linear's weight), 16-byte aligned; proj_b: fp32 [H*D] or NULL.
 * The attention output is rounded to the attention dtype before the
 * projection, as the two-step composition does.  Only the wave kernel's
 * case with every head in one workgroup is fused: 16-bit q/k/v, head_dim 32,
 * H <= 4 and H * M <= 192; other shapes return AFF_ERR_UNSUPPORTED (the
 * caller then runs aff_nbhd_attn_fwd and its own projection).  lse is
 * written when args->lse is set.
 * ------------------------------------------------------------------------ */
aff_status aff_nbhd_attn_proj_fwd(const aff_nbhd_attn_args *args, const void *proj_w, const float *proj_b,
                                  aff_stream_t stream);
/* ------------------------------------------------------------------------ *
 * Neighbourhood (cluster) flash attention, backward.
 *
 * Replaces: launch_flash_nbhood_attn_bwd()  src/layers/kernels/local_attn.py:711-840
 *           kernels _nbhood_attn_bwd_preprocess / _nbhood_attn_bwd_internal
 *           local_attn.py:350-606 (FlashLocalAttentionFunction.backward :911-936)
 *
 * With Delta = sum_d out * dout over each (b, h, n) row (out = the forward
 * output), and for every valid neighbour j of the row (valid as in the
 * forward; masked and out-of-range neighbours get no gradient):
 *   p_j  = exp(s_j - lse),  s_j = scale <q, k_j> + bias_j
 *   dS_j = p_j (<dout, v_j> - Delta)
 *   dq   = scale (sum_j dS_j k_j + dS_blank blank_k)
 *   dk[idx_j] += scale dS_j q,   dv[idx_j] += p_j dout
 *   dbias[b, h, n, j] = dS_j
 *   dtable[row_j, h] += dS_j  (bias modes 2 and 4: row_j the table row the forward read)
 *   dblank_k[h] += scale dS_blank q,  dblank_v[h] += p_blank dout
 * The scattered sums are formed without floating-point atomics, each in a
 * fixed order (the (b, n, j) order of the contributing pairs), so the
 * result is bitwise reproducible.
 *
 * fwd: the forward call's arguments; fwd.out must be the forward output and
 * fwd.lse its LSE (both required); fwd.ws is not used.  Bias modes 0, 1, 2
 * and 4 (mode 3 returns AFF_ERR_UNSUPPORTED).
 * dout / dq / dk / dv: [B, H, N, D] in fwd.dtype with element strides and a
 * unit stride on D (16-byte aligned rows).  dk / dv rows no pair points at
 * are written as zeros.
 * dbias: [B, H, N, M] fp32 contiguous, or NULL.  dtable: [table_rows, H] fp32
 * contiguous (modes 2 and 4), or NULL.  dblank_k / dblank_v: [H, D] fp32,
 * both set (when the forward had blank tokens) or both NULL.
 * ws: aff_nbhd_attn_bwd_workspace_bytes() bytes, 256-byte aligned.
 * ------------------------------------------------------------------------ */
typedef struct aff_nbhd_attn_bwd_args {
    aff_nbhd_attn_args fwd;
    const void *dout; int64_t do_sb, do_sh, do_sn;
    void *dq; int64_t dq_sb, dq_sh, dq_sn;
    void *dk; int64_t dk_sb, dk_sh, dk_sn;
    void *dv; int64_t dv_sb, dv_sh, dv_sn;
    float *dbias;
    float *dtable;
    float *dblank_k;
    float *dblank_v;
    void *ws; size_t ws_bytes;
} aff_nbhd_attn_bwd_args;

size_t aff_nbhd_attn_bwd_workspace_bytes(const aff_nbhd_attn_bwd_args *args);
aff_status aff_nbhd_attn_bwd(const aff_nbhd_attn_bwd_args *args, aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Weighted neighbour features (the AFF downsampling merge).
 *
 * Replaces: weighted_features() / WeightedFeaturesFunction
 *           src/layers/kernels/weighted_features.py:401-434, kernel :30-111
 *
 *   out[b, i, ic, c] = sum_m weights[b, i, m, ic] * feat[b, idx[b, i, m], c]
 *
 * weights [B, Nout, M, IC] (w_dtype, strides w_sb, w_sn, w_sm, w_sic);
 * feat [B, Nsrc, C] (f_dtype, unit stride on C); nbhd_idx [B, Nout, M]
 * int32/int64 with unit stride on M; out [B, Nout, IC, C] in f_dtype with
 * unit stride on C.  fp32 accumulation.  Indices outside [0, Nsrc)
 * contribute nothing.
 * ------------------------------------------------------------------------ */
aff_status aff_weighted_features_fwd(const void *weights, int w_dtype, int64_t w_sb, int64_t w_sn,
                                     int64_t w_sm, int64_t w_sic,
                                     const void *feat, int f_dtype, int64_t f_sb, int64_t f_sn,
                                     const void *nbhd_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn,
                                     int B, int Nout, int Nsrc, int M, int C, int IC,
                                     void *out, int64_t o_sb, int64_t o_sn, int64_t o_sic,
                                     aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Weighted neighbour features, backward.
 *
 * Replaces: WeightedFeaturesFunction.backward  src/layers/kernels/weighted_features.py:421-430,
 *           kernels :164-398; WeightedGatherFunction.backward (weighted_gather.py:349-361,
 *           kernels :127-326) as the IC = 1 case.
 *
 *   d_weights[b, i, m, ic] = sum_c dout[b, i, ic, c] * feat[b, idx[b, i, m], c]
 *   d_feat[b, r, c] = sum over (i, m) with idx[b, i, m] = r of
 *                     sum_ic weights[b, i, m, ic] * dout[b, i, ic, c]
 * dout [B, Nout, IC, C] in f_dtype (strides do_sb, do_sn, do_sic; unit stride
 * on C); weights / feat / nbhd_idx as in the forward.  d_weights: [B, Nout, M,
 * IC] contiguous in dw_dtype, or NULL; d_feat: [B, Nsrc, C] contiguous in
 * f_dtype, or NULL.  Indices outside [0, Nsrc) contribute nothing and get
 * d_weights 0.  IC <= 8.  d_feat is a fixed-order sum (the (b, i, m) order of
 * the entries), with no atomics: bitwise reproducible.  ws:
 * aff_weighted_features_bwd_workspace_bytes(B, Nout, Nsrc, M) bytes, 256-byte
 * aligned (only needed for d_feat).
 * ------------------------------------------------------------------------ */
size_t aff_weighted_features_bwd_workspace_bytes(int B, int Nout, int Nsrc, int M);
aff_status aff_weighted_features_bwd(const void *dout, int64_t do_sb, int64_t do_sn, int64_t do_sic,
                                     const void *weights, int w_dtype, int64_t w_sb, int64_t w_sn,
                                     int64_t w_sm, int64_t w_sic,
                                     const void *feat, int f_dtype, int64_t f_sb, int64_t f_sn,
                                     const void *nbhd_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn,
                                     int B, int Nout, int Nsrc, int M, int C, int IC,
                                     void *d_weights, int dw_dtype, void *d_feat,
                                     void *ws, size_t ws_bytes, aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Weighted gather: the IC = 1 case of the above.
 *
 * Replaces: weighted_gather() / WeightedGatherFunction
 *           src/layers/kernels/weighted_gather.py:329-364, kernel :21-102
 *
 *   out[b, i, c] = sum_m weights[b, i, m] * feat[b, idx[b, i, m], c]
 * ------------------------------------------------------------------------ */
aff_status aff_weighted_gather_fwd(const void *nbhd_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn,
                                   const void *weights, int w_dtype, int64_t w_sb, int64_t w_sn,
                                   const void *feat, int f_dtype, int64_t f_sb, int64_t f_sn,
                                   int B, int Nout, int Nsrc, int M, int C,
                                   void *out, int64_t o_sb, int64_t o_sn, aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Softmax-distance merge: weighted_gather with weights computed in-kernel.
 *
 * Replaces the composition knn -> softmax(-d / tau) -> weighted_gather on
 * features and on coordinates (reference kernels weighted_gather.py:21-102,
 * upsample_feature_shepard geometry.py:97-167 for the gather pattern):
 *
 *   d_m = sqrt(fl(fl(dx*dx) + fl(dy*dy))),  (dx, dy) = qpos[b,i] - spos[b, idx_m]
 *   w_m = softmax_m(-d_m / tau)
 *   out[b, i, :] = sum_m w_m feat[b, idx_m, :],  out_pos[b, i, :] = sum_m w_m spos[b, idx_m, :]
 *
 * query_pos [B, Nout, 2], src_pos [B, Nsrc, 2] fp32 (unit coordinate stride);
 * feat [B, Nsrc, C] (C % 8 == 0, 16-byte aligned rows); nbhd_idx [B, Nout, K]
 * (K <= 128, unit stride on K); out [B, Nout, C] in f_dtype; out_pos
 * [B, Nout, 2] fp32 and out_weights [B, Nout, K] fp32 contiguous may be NULL.
 * Indices outside [0, Nsrc) get weight 0.
 * ------------------------------------------------------------------------ */
aff_status aff_softmax_merge_fwd(const float *query_pos, int64_t q_sb, int64_t q_sn,
                                 const float *src_pos, int64_t s_sb, int64_t s_sn,
                                 const void *feat, int f_dtype, int64_t f_sb, int64_t f_sn,
                                 const void *nbhd_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn,
                                 int B, int Nout, int Nsrc, int K, int C, float tau,
                                 void *out, int64_t o_sb, int64_t o_sn,
                                 float *out_pos, int64_t op_sb, int64_t op_sn, float *out_weights,
                                 aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Deformable attention over point clouds with in-kernel exact K-NN.
 *
 * Replaces: fused_knn_deformable_cross_attention / _self_attention
 *           src/layers/kernels/fused_deform_attn.py:4063-4119, launchers
 *           :2387-2654, kernels :842-1011 (self) and :1188-1335 (cross);
 *           and the multi-level composition knn(k=3) + inverse_distance_weighting
 *           (src/utils/geometry.py:40-53) + MSDETRPC (msdetrpc.py:25-109).
 *
 * For every (b, q, h) and sample s = (l, p), l < L levels, p < P points:
 *   loc  = query_pos[b, q] + offsets[b, q, h, l, p, :]            (fp32)
 *   the K points of level l nearest to loc, exact, ties to the lower index
 *   (d2 = fl(fl(dx*dx) + fl(dy*dy)));  fewer than K points -> all of them
 *   mode AFF_DEFORM_SHEPARD: w_j = e_j / (sum e + 1e-8),
 *        e_j = exp(lg_j - max lg),  lg_j = -max(power, 1e-6) * (sqrt(d2_j) + 1e-6)
 *   mode AFF_DEFORM_IDW:     w_j = u_j / (sum u + 1e-12),  u_j = 1 / (d2_j^power + 1e-10)
 *   out[b, q, h, :] = sum_s attn[b, q, h, l, p] * sum_j w_j * values[b, start[l] + idx_j, h, :]
 *
 * kv_pos [B, Ntot, 2] fp32 with level l in rows [level_start[l], level_start[l+1])
 * (level_start[0] = 0, non-decreasing, L <= AFF_DEFORM_MAX_LEVELS; self-attention
 * passes query_pos as kv_pos with L = 1).  offsets [B, Nq, H, L, P, 2] and attn
 * [B, Nq, H, L, P] with strides (sb, sn, sh) and the (L, P[, 2]) block contiguous,
 * any of fp32/fp16/bf16.  values [B, Ntot, H, C] and out [B, Nq, H, C] in `dtype`
 * with strides (sb, sn, sh), unit stride on C, C % 8 == 0, 16-byte aligned rows.
 * power: device pointer to one fp32 (no host synchronisation).  1 <= K <= 8,
 * L * P <= 32.  knn_idx (int32, level-local index, -1 if missing) and knn_d2
 * ([B, Nq, H, L, P, K] contiguous) may be NULL.  ws: aff_deform_workspace_bytes().
 * ------------------------------------------------------------------------ */
#define AFF_DEFORM_MAX_LEVELS 8
enum { AFF_DEFORM_SHEPARD = 0, AFF_DEFORM_IDW = 1 };

typedef struct aff_deform_args {
    int mode;
    int B, Nq, H, L, P, K, C;
    const float *query_pos; int64_t qp_sb, qp_sn;
    const float *kv_pos; int64_t kp_sb, kp_sn;
    int level_start[AFF_DEFORM_MAX_LEVELS + 1];
    const void *offsets; int off_dtype; int64_t off_sb, off_sn, off_sh;
    const void *attn; int attn_dtype; int64_t at_sb, at_sn, at_sh;
    int dtype; const void *values; int64_t v_sb, v_sn, v_sh;
    const float *power;
    void *out; int64_t o_sb, o_sn, o_sh;
    int32_t *knn_idx;
    float *knn_d2;
} aff_deform_args;

size_t aff_deform_workspace_bytes(const aff_deform_args *args);
aff_status aff_deform_fwd(const aff_deform_args *args, void *ws, size_t ws_bytes, aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Distance-softmax weights from given neighbour indices, optionally gathered.
 *
 * Replaces: fused_deformable_attention()  fused_deform_attn.py:694-718,
 *           launcher :503-571, kernel :79-231                  (eps_mode 0)
 *           mssample()  src/layers/kernels/mssample.py:452-478,
 *           launcher :300-342, kernel :17-125                  (eps_mode 1)
 *
 *   dist_k = eps_mode == 0 ? sqrt(d2_k) + 1e-6 : sqrt(d2_k + 1e-6),
 *            d2_k = |sampling_locs[b, n] - kv_pos[b, idx[b, n, k]]|^2 over D <= 4 dims
 *   w_k    = e_k / (sum e + 1e-8),  e_k = exp(-max(power, 1e-6) * dist_k - max)
 *   weights[b, n, k] = w_k                                     (if weights != NULL)
 *   out[b, n, :] = attn[b, n] * sum_k w_k values[b, idx_k, :]   (if out != NULL;
 *                  attn NULL means 1)
 * Indices outside [0, Nkv) get weight 0.  K <= 64.  power is a device scalar.
 * values / out: `dtype`, C % 8 == 0, 16-byte aligned rows, unit stride on C.
 * ------------------------------------------------------------------------ */
aff_status aff_deform_sample_fwd(int eps_mode, const float *sampling_locs, int64_t l_sb, int64_t l_sn,
                                 const float *kv_pos, int64_t k_sb, int64_t k_sn,
                                 const void *nb_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn,
                                 const float *power, int B, int N, int Nkv, int K, int D,
                                 const void *attn, int attn_dtype, int64_t a_sb, int64_t a_sn,
                                 const void *values, int dtype, int64_t v_sb, int64_t v_sn, int C,
                                 void *out, int64_t o_sb, int64_t o_sn,
                                 void *weights, int w_dtype, int64_t w_sb, int64_t w_sn,
                                 aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Multi-slot deformable gather.
 *
 * Replaces: MSDETRPCFunction  src/layers/kernels/msdetrpc.py:372-390,
 *           launcher :305-325, kernel :25-109
 *
 *   out[b, n, c] = sum_m sum_k attn[b, n, m] * nn_weight[b, n, m, k] * val[b, nn_idx[b, n, m, k], c]
 *
 * nn_idx / nn_weight [B, N, M, K] (strides sb, sn, sm; unit stride on K);
 * attn [B, N, M] (unit stride on M); val [B, Nval, C] and out [B, N, C] in
 * `dtype`, C % 8 == 0, 16-byte aligned rows.  Indices outside [0, Nval)
 * contribute nothing.
 * ------------------------------------------------------------------------ */
aff_status aff_msdetrpc_fwd(const void *nn_idx, int idx_is_i64, int64_t i_sb, int64_t i_sn, int64_t i_sm,
                            const void *nn_weight, int w_dtype, int64_t w_sb, int64_t w_sn, int64_t w_sm,
                            const void *attn, int a_dtype, int64_t a_sb, int64_t a_sn,
                            const void *val, int dtype, int64_t v_sb, int64_t v_sn,
                            int B, int N, int M, int K, int Nval, int C,
                            void *out, int64_t o_sb, int64_t o_sn, aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Backward of the deformable gathers (all three forward entry points above).
 *
 * Replaces: fused_knn_deform_cross_attn_backward / _self_attn_backward
 *           src/layers/kernels/fused_deform_attn.py:2661-2930 (kernels
 *           :1521-2386), FusedKNNDeform{Self,Cross}AttnFunction.backward
 *           :4002, :4041;  fused_deform_attn_backward :574-650 (kernel
 *           :253-500), FusedDeformAttnFunction.backward :679;
 *           mssample_backward  mssample.py:345-399 (kernel :142-298);
 *           launch_msdetrpc_backward  msdetrpc.py:328-369 (kernels :133-300).
 *
 * One row r = (b, q, h) of dout [B, Q, H, C] holds S samples of K neighbours:
 *   out[r] = sum_s attn[r, s] * sum_j w[r, s, j] * values[b, row(s, j), h]
 * row(s, j) = level_start[s / P] + idx[r, s, j]; a pair is valid when
 * idx >= 0 and row < level_start[s / P + 1] (invalid pairs carry no weight).
 * Weights by `mode` (the forward's formulas, recomputed from positions:
 * loc = loc[b, q] + offsets[r, s] (offsets NULL = 0), d2 = sum_d fl(diff_d^2),
 * diff = loc - kv_pos[b, row], p = max(power, 1e-6)):
 *   AFF_DEFORM_BWD_SHEPARD  softmax(-p (sqrt(d2) + 1e-6)), aff_deform_fwd SHEPARD
 *   AFF_DEFORM_BWD_IDW      IDW on d2 with the raw power, aff_deform_fwd IDW
 *   AFF_DEFORM_BWD_SAMPLE   softmax(-p (sqrt(d2) + 1e-6)), aff_deform_sample_fwd eps 0
 *   AFF_DEFORM_BWD_SAMPLE_SQ softmax(-p sqrt(d2 + 1e-6)), aff_deform_sample_fwd eps 1
 *   AFF_DEFORM_BWD_GIVEN    weights[r, s, j] as given (aff_msdetrpc_fwd)
 * With g_j = dL/dw_j (= attn * <dout[r], values[b, row_j, h]>, or d_w_in when
 * values is NULL), the distance modes follow the reference's chain rule:
 * the softmax backward dlg_j = w_j (g_j - sum_i w_i g_i) treats the 1e-8 of
 * the denominator as absent; d(loc) = sum_j dist'_j (diff_j) with
 *   SHEPARD   -p dlg_j diff_j / (sqrt(d2_j) + 1e-6)
 *   SAMPLE    -p dlg_j diff_j / max(sqrt(d2_j) + 1e-6 - 1e-6, 1e-8)
 *   SAMPLE_SQ -p dlg_j diff_j / (sqrt(d2_j + 1e-6) + 1e-8)
 *   IDW       2 diff_j dL/du_j du_j/dd2_j,  dL/du_j = (g_j - sum_i w_i g_i) / (sum u + 1e-12)
 * and d(kv_pos[b, row_j]) gets the negated pair term; d_power = sum over
 * pairs of dlg_j (-dist_j) (IDW: dL/du_j du_j/dpower, 0 where d2 == 0).
 *
 * Every scattered sum (d_values, d_kv_pos, d_power) is a fixed-order gather
 * over pairs bucketed by a stable sort: the results are bitwise reproducible.
 * Layouts: loc [B, Q, D] fp32 (D <= 4); offsets [B, Q, H, S, D] with (S, D)
 * contiguous; idx [B, Q, H, S, K] int32/int64 with (S, K) contiguous; attn
 * [B, Q, H, S] (S contiguous) or NULL = 1; weights / d_w_in [B, Q, H, S, K];
 * kv_pos [B, Nkv, D] fp32; values [B, Nkv, H, C] and dout [B, Q, H, C] in
 * `dtype`, unit stride on C, C % 8 == 0, C <= 2048, 16-byte aligned rows.
 * Outputs (each NULL when not wanted, contiguous): d_loc [B, Q, H, S, D]
 * fp32 (d_offsets; its sum over (h, s) is d(loc)), d_attn [B, Q, H, S] fp32,
 * d_weights [B, Q, H, S, K] fp32 (GIVEN), d_kv_pos [B, Nkv, D] fp32,
 * d_values [B, Nkv, H, C] in `dtype`, d_power one fp32.  K <= 16,
 * B * Q * H * S * K < 2^31.  ws: aff_deform_bwd_workspace_bytes().
 * ------------------------------------------------------------------------ */
enum {
    AFF_DEFORM_BWD_SHEPARD = 0,
    AFF_DEFORM_BWD_IDW = 1,
    AFF_DEFORM_BWD_SAMPLE = 2,
    AFF_DEFORM_BWD_SAMPLE_SQ = 3,
    AFF_DEFORM_BWD_GIVEN = 4
};

typedef struct aff_deform_bwd_args {
    int mode;
    int B, Q, H, S, K, C, D, P, Nkv;
    int level_start[AFF_DEFORM_MAX_LEVELS + 1];
    const float *loc; int64_t loc_sb, loc_sn;
    const void *offsets; int off_dtype; int64_t off_sb, off_sn, off_sh;
    const float *kv_pos; int64_t kp_sb, kp_sn;
    const void *idx; int idx_is_i64; int64_t i_sb, i_sn, i_sh;
    const void *attn; int attn_dtype; int64_t at_sb, at_sn, at_sh;
    const void *weights; int w_dtype; int64_t w_sb, w_sn, w_sh;
    int dtype;
    const void *values; int64_t v_sb, v_sn, v_sh;
    const void *dout; int64_t do_sb, do_sn, do_sh;
    const float *d_w_in; int64_t dwi_sb, dwi_sn, dwi_sh;
    const float *power;
    float *d_loc;
    float *d_attn;
    float *d_weights;
    float *d_kv_pos;
    void *d_values;
    float *d_power;
} aff_deform_bwd_args;

size_t aff_deform_bwd_workspace_bytes(const aff_deform_bwd_args *args);
aff_status aff_deform_bwd(const aff_deform_bwd_args *args, void *ws, size_t ws_bytes, aff_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Neighbourhood index construction of the encoder's BasicLayer.
 *
 * Replaces the torch gathers of BasicLayer.forward  src/layers/aff.py:452-465
 * (member gather, padding-mask gather, relative-position table index).
 *
 * For token n of image b and slot j < nnc * m, with c = nearest[b, n, j / m]
 * and i = j % m:
 *   out_member[b, n, j] = members[b, c, i]
 *   out_mask[b, n, j]   = cmask[b, c, i] != 0          (1 when cmask is NULL)
 *   out_pe[b, n, j]     = trunc(rel_y * (2W + 1) + rel_x), fp32, no contraction,
 *                         rel = clamp(pos[b, member] - (pos[b, n] - W), 0, 2W)
 * nearest [B, N, nnc] (int32/int64, strides n_sb, n_sn, unit on the last dim),
 * members [B, K, m] (int32/int64, strides m_sb, m_sk), cmask [B, K, m] uint8
 * (strides c_sb, c_sk) or NULL, pos [B, N, 2] fp32 (strides p_sb, p_sn).
 * Outputs are [B, N, nnc * m] contiguous: out_member int32/int64
 * (out_is_i64), out_mask uint8 or NULL, out_pe int32/int64 or NULL.  A
 * cluster id outside [0, K) or a member outside [0, N) yields member 0 and
 * mask 0.  W = rel_width (127 in the reference).
 * ------------------------------------------------------------------------ */
aff_status aff_cluster_members(const void *nearest, int near_is_i64, int64_t n_sb, int64_t n_sn,
                               const void *members, int mem_is_i64, int64_t m_sb, int64_t m_sk,
                               const uint8_t *cmask, int64_t c_sb, int64_t c_sk,
                               const float *pos, int64_t p_sb, int64_t p_sn,
                               int B, int N, int K, int nnc, int m, int rel_width,
                               void *out_member, int out_is_i64, uint8_t *out_mask,
                               void *out_pe, int pe_is_i64, aff_stream_t stream);

/* ---------------------------------------------------------------------------
 * aff_layer_norm_fwd — LayerNorm over the last dimension, forward.
 * Replaces the encoder's nn.LayerNorm calls on token rows (reference
 * src/layers/aff.py:96,108 block norms, :296 merge norm, :494 downsample
 * norm, :726 stage norms).
 *
 * x [rows, C] (dtype x_dtype, row stride x_rs elements, unit channel stride)
 * -> y [rows, C] (y_dtype, row stride y_rs): fp32 mean and biased variance,
 * y = (x - mean) * rsqrt(var + eps) * weight + bias (weight / bias fp32 [C]
 * or NULL, 16-byte aligned).  C % 8 == 0, C <= 4096, x / y and their row
 * strides 16-byte aligned.  y_dtype may differ from x_dtype (an autocast consumer's dtype).
 * ------------------------------------------------------------------------ */
aff_status aff_layer_norm_fwd(const void *x, int x_dtype, int64_t x_rs, void *y, int y_dtype, int64_t y_rs,
                              const float *weight, const float *bias, int64_t rows, int C, float eps,
                              aff_stream_t stream);

/* ---------------------------------------------------------------------------
 * aff_layer_norm_map_fwd — LayerNorm over the channels of a [B, C, H, W] map,
 * with the masked patch embedding's mask and activation fused.
 * Replaces LayerNorm2dImages + GELU after a masked convolution, and the
 * final token LayerNorm of the patch embedding (reference
 * src/layers/aff.py:514-526, 610-632).
 *
 * x [B, C, H, W] contiguous (x_dtype).  Per pixel: v = x * keep[b, token]
 * when keep (fp32 [B, (H / cell) * (W / cell)], token = (y / cell) *
 * (W / cell) + x / cell) is given, then LayerNorm over C (fp32 statistics,
 * weight / bias fp32 [C] or NULL), then the exact-erf GELU when gelu != 0.
 * Output y is [B, C, H, W] (token_major = 0) or [B, H * W, C]
 * (token_major = 1), contiguous, y_dtype.  C <= 64.
 * ------------------------------------------------------------------------ */
aff_status aff_layer_norm_map_fwd(const void *x, int x_dtype, void *y, int y_dtype, const float *weight,
                                  const float *bias, const float *keep, int cell, int B, int C, int H, int W,
                                  int token_major, int gelu, float eps, aff_stream_t stream);

/* ---------------------------------------------------------------------------
 * Space-filling-curve ordering of tokens (the balanced clustering's sort keys).
 *
 * Replaces the key computation and sort of space_filling_cluster
 * (src/utils/geometry.py:199-288) and calculate_peano_order /
 * calculate_hilbert_order (geometry.py:322-460).
 *
 * aff_sfc_curve_keys: keys[b, n] (fp32) of pos[b, n] (fp32 (x, y), strides
 * p_sb, p_sn, unit stride on the coordinate) along
 *   AFF_SFC_SCANLINE  rows alternating in direction: id = trunc(x + y * w),
 *                     key = (row odd ? w - 1 - col : col) + row * w
 *   AFF_SFC_PEANO / AFF_SFC_HILBERT  `levels` base-3 / base-2 digit levels;
 *                     digit_l = floor(rem * inv_h[l]), rem = fmod(rem, cur_h[l])
 *                     (cur_h[l] the reference's h / base^(l+1) rounded to fp32,
 *                     inv_h[l] = 1 / cur_h[l] in fp32), digits outside the
 *                     canvas clamped; first_w > 0 selects the reference's wide
 *                     first level (Peano only); key = order[L-1] + sum_l
 *                     order[l] * level_scale[l] in fp32, in order of l.
 * aff_sfc_anchor_keys: keys[b, n] = rank * (max ratio + 1) + ratio with the
 *   patch of pos = (floor(x / plw), floor(y / plh)), cell = px + py * npw
 *   (clamped to [0, ncell)), rank = cell_rank[cell], ratio = |pos - prev|^2
 *   / (|pos - next|^2 + 1e-5), prev / next = prev_c / next_c[rank] (fp32
 *   [ncell, 2], the centres of the neighbouring patches on the curve), the
 *   maximum over all b, n.  ws: aff_sfc_anchor_workspace_bytes(B, N).
 * aff_sfc_argsort: ranking[b, i] (int64) = the index of the token of rank i in
 *   row b of keys [B, N] (fp32, contiguous), ascending, ties to the lower
 *   index.  ws: aff_sfc_argsort_workspace_bytes(B, N).  Not for HIP graph
 *   capture: its radix sort clears state with hipMemsetAsync.
 * ------------------------------------------------------------------------ */
#define AFF_SFC_MAX_LEVELS 16
enum { AFF_SFC_SCANLINE = 0, AFF_SFC_PEANO = 1, AFF_SFC_HILBERT = 2 };

typedef struct aff_sfc_curve_args {
    const float *pos; int64_t p_sb, p_sn;
    int B, N, curve, w, levels, first_w;
    float cur_h[AFF_SFC_MAX_LEVELS];
    float inv_h[AFF_SFC_MAX_LEVELS];
    float level_scale[AFF_SFC_MAX_LEVELS];
    float *keys;
} aff_sfc_curve_args;

typedef struct aff_sfc_anchor_args {
    const float *pos; int64_t p_sb, p_sn;
    int B, N;
    float plw, plh;
    int npw, ncell;
    const int *cell_rank;
    const float *prev_c;
    const float *next_c;
    float *keys;
} aff_sfc_anchor_args;

aff_status aff_sfc_curve_keys(const aff_sfc_curve_args *args, aff_stream_t stream);
size_t aff_sfc_anchor_workspace_bytes(int B, int N);
aff_status aff_sfc_anchor_keys(const aff_sfc_anchor_args *args, void *ws, size_t ws_bytes, aff_stream_t stream);
size_t aff_sfc_argsort_workspace_bytes(int B, int N);
aff_status aff_sfc_argsort(const float *keys, int B, int N, int64_t *ranking, void *ws, size_t ws_bytes,
                           aff_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* AFFMAE_H */
