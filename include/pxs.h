/*
 * pxs.h - C ABI of the MI355X (gfx950) sparse-voxel kernels.
 *
 * Conventions
 *   - Every pointer argument named in "device" terms points to HBM; shapes are
 *     plain integers; `stream` is a hipStream_t (NULL = default stream).
 *   - Calls return PXS_OK (0) or an error code and record a message readable
 *     with pxs_last_error() (thread-local).  Host-checkable argument errors
 *     are reported before anything is enqueued.
 *   - Calls are asynchronous on `stream` unless stated; none of them allocate
 *     device memory: scratch comes from a caller-provided workspace sized by
 *     the matching *_workspace_bytes query.
 *   - Coordinates are int32 rows (batch, x, y, z).  Features are row-major
 *     [rows, channels].  PXS_BF16 data is stored as raw bfloat16 bit
 *     patterns (uint16); arithmetic accumulates in fp32.
 *
 * Each entry point names the reference interface it replaces; paths are
 * relative to the Pixal3D.cpp tree.
 */
#ifndef PXS_H
#define PXS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PXS_OK 0
#define PXS_ERR_ARG 1  /* invalid argument (host-checked) */
#define PXS_ERR_HIP 2  /* HIP runtime error */
#define PXS_ERR_DATA 3 /* data error detected on the device (validation) */

#define PXS_F32 0
#define PXS_BF16 1

/* Largest batch count and per-axis spatial extent the voxel key encodes. */
#define PXS_MAX_EXTENT 32768

#define PXS_ACT_NONE 0
#define PXS_ACT_GELU_TANH 1
#define PXS_ACT_SILU 2

const char * pxs_last_error(void);
int pxs_version(void);

/* ---- a1, a2: validation, voxel hash, neighbor maps -------------------------- */

/* Bytes of the open-addressing voxel hash for n rows. */
size_t pxs_voxel_hash_bytes(int64_t n);

/* Build the lock-free voxel hash of n coordinate rows into `table`
 * (pxs_voxel_hash_bytes(n) bytes).  Each slot keeps the smallest row that
 * inserted its key, so a duplicate coordinate is visible to
 * pxs_sparse_validate.  Replaces the std::unordered_map builds of
 * src/sparse.cpp:1017-1022 and src/slat_decoder.cpp:630-635. */
int pxs_voxel_hash_build(const int32_t * coords, int64_t n, void * table, void * stream);

/* SparseTensorF32::valid (src/sparse.cpp:241-335) on the device.  Needs the
 * hash of the same coords.  Writes *status (device int64) = first failing
 * row * 8 + code, or INT64_MAX when valid; code 4 = outside shape,
 * 5 = duplicate, 6 = not contiguous by batch, 7 = non-finite feature (the
 * reference's check order at one row).  feats may be NULL to skip code 7. */
int pxs_sparse_validate(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                        int sz, int dtype, const void * feats, int channels,
                        const void * table, int64_t * status, void * stream);

/* The reference's message for a validation code (src/sparse.cpp:249-330). */
const char * pxs_validation_message(int code);

/* Dense 3x3x3 neighbor map (src/slat_decoder.cpp:609-668): nbr[k * n + p] is
 * the row of voxel (b, x+kd-1, y+kh-1, z+kw-1), k = kd*9 + kh*3 + kw, or n
 * when absent.  masks (nullable) receives bit k set when offset k is present. */
int pxs_neighbor_map_k3(const int32_t * coords, int64_t n, const void * table, int32_t * nbr,
                        uint32_t * masks, void * stream);

/* Compacted per-offset pair lists from a dense map: for each k ascending,
 * (input row, output row) pairs with output rows ascending; offsets28
 * (device int64[28]) bounds the lists.  pair_in/pair_out hold up to 27*n. */
size_t pxs_neighbor_pairs_workspace_bytes(int64_t n);
int pxs_neighbor_pairs(const int32_t * nbr, int64_t n, int32_t * pair_in, int32_t * pair_out,
                       int64_t * offsets28, void * workspace, void * stream);

/* ---- a3: submanifold convolution ------------------------------------------- */

/* sparse_submanifold_conv3d (src/sparse.cpp:999-1055): y[p] = sum over present
 * k of W_k x[nbr[k][p]] + bias.  weight [27, cout, cin] (compact-v1 layout),
 * bias fp32 [cout].  dtype PXS_F32: x, weight, y fp32 (fp32 MFMA);
 * PXS_BF16: x, weight, y bf16 with fp32 accumulation.  masks (from
 * pxs_neighbor_map_k3) let tiles skip absent offsets; NULL processes all 27.
 * Output-stationary: each output row is written once, no atomics. */
int pxs_subm_conv3d(int dtype, const void * x, int64_t n, int cin, const void * weight,
                    const float * bias, int cout, const int32_t * nbr, const uint32_t * masks,
                    void * y, void * stream);

/* ---- a4, a15: stride-2 topology, strided conv, mean downsample -------------- */

/* Output topology of a factor-2 reduction: the unique (b, x/2, y/2, z/2) in
 * lexicographic order (the coordinates sparse_downsample_mean emits,
 * src/sparse.cpp:553-593).  out_coords holds up to n rows; child_map is
 * [8][n] (offset-major, leading dimension n): child c = (x&1) + 2(y&1) +
 * 4(z&1) of output q is input row child_map[c * n + q], or -1.  *m_out
 * (device int64) receives the output row count. */
size_t pxs_downsample_workspace_bytes(int batch_size, int sx, int sy, int sz);
int pxs_downsample_s2_topology(const int32_t * coords, int64_t n, int batch_size, int sx,
                               int sy, int sz, int32_t * out_coords, int32_t * child_map,
                               int64_t * m_out, void * workspace, void * stream);

/* Stride-2 SparseConv3d with a 2x2x2 kernel (no reference counterpart; the
 * contract is documented with the topology above): y[q] = sum over present
 * children c of W_c x[child] + bias, weight [8, cout, cin].  ld_map is the
 * leading dimension of child_map (the n passed to the topology call), m the
 * output rows. */
int pxs_sparse_conv3d_s2(int dtype, const void * x, int64_t n_in, int cin, const void * weight,
                         const float * bias, int cout, const int32_t * child_map, int64_t ld_map,
                         int64_t m, void * y, void * stream);

/* sparse_downsample_mean features for factor 2 (src/sparse.cpp:536-602):
 * each output is the mean of its children summed in input-row order. */
int pxs_downsample_mean_s2(int dtype, const void * x, int channels, const int32_t * child_map,
                           int64_t ld_map, int64_t m, void * y, void * stream);

/* ---- a5: channel to spatial ---------------------------------------------------- */

/* sparse_channel_to_spatial with factor 2 (src/sparse.cpp:604-702).
 * x [n, 8*c_out]; subdivision (nullable, fp32 [n, 8]) selects children > 0.
 * Output rows are parent-major, child ascending; out_coords and y hold up to
 * 8n rows; *m_out (device int64) receives the count. */
size_t pxs_channel_to_spatial_workspace_bytes(int64_t n);
int pxs_channel_to_spatial(int dtype, const int32_t * coords, int64_t n, const void * x,
                           int channels, const float * subdivision, int32_t * out_coords,
                           void * y, int64_t * m_out, void * workspace, void * stream);

/* ---- a6: sparse linear --------------------------------------------------------- */

/* sparse_linear / varlen_linear (src/sparse.cpp:337-488): y = x W^T + bias,
 * weight [cout, cin] row-major, then an optional activation (PXS_ACT_*,
 * the GELU-tanh of src/sparse_transformer.cpp:123-134 or the SiLU of
 * src/slat_decoder.cpp:68-78).  bias may be NULL. */
int pxs_linear(int dtype, const void * x, int64_t rows, int cin, const void * weight,
               const float * bias, int cout, int act, void * y, void * stream);

/* Linear whose epilogue applies the adaLN gate and the residual add of
 * src/sparse_transformer.cpp:229-235 (gate_in_place + add_in_place):
 * residual[r, o] += (block_mod[off + o] + time_mod[b(r) * 6 * cout + off + o])
 *                   * (x W^T + bias)[r, o], with b(r) = coords[r * 4].
 * residual is fp32 and updated in place. */
int pxs_linear_gate_residual(int dtype, const void * x, int64_t rows, int cin,
                             const void * weight, const float * bias, int cout,
                             const int32_t * coords, const float * block_mod,
                             const float * time_mod, int gate_offset, float * residual,
                             void * stream);

/* ---- a10-a12: row-wise normalisation and position embedding ------------------- */

/* sparse_layer_norm (src/sparse.cpp:490-534); gamma/beta both NULL or both set.
 * x and y may have different dtypes (fp32 residual -> bf16 GEMM input). */
int pxs_layer_norm(int x_dtype, const void * x, int64_t rows, int channels, float eps,
                   const float * gamma, const float * beta, int y_dtype, void * y, void * stream);

/* Layer norm without affine followed by the adaLN modulation of
 * src/sparse_transformer.cpp:71-99: y = ln(x) * (1 + scale) + shift with
 * scale/shift = block_mod[off (+C) + c] + time_mod[b(r) * 6C + off (+C) + c]. */
int pxs_layer_norm_modulate(int x_dtype, const void * x, int64_t rows, int channels, float eps,
                            const int32_t * coords, const float * block_mod,
                            const float * time_mod, int mod_offset, int y_dtype, void * y,
                            void * stream);

/* sparse_multihead_rms_norm / varlen_multihead_rms_norm
 * (src/sparse.cpp:919-997).  Rows have stride ld_x / ld_y elements. */
int pxs_mh_rms_norm(int dtype, const void * x, int64_t ld_x, int64_t rows, int heads,
                    int head_dim, const float * gamma, void * y, int64_t ld_y, void * stream);

/* sparse_rotary_position_embedding (src/sparse.cpp:861-917). */
int pxs_rope(int dtype, const int32_t * coords, const void * x, int64_t ld_x, int64_t rows,
             int heads, int head_dim, float freq_min, float freq_base, void * y, int64_t ld_y,
             void * stream);

/* Fused attention prologue: split qkv [rows, 3C] into q, k, v [rows, C],
 * applying the per-head RMS norm (q_gamma/k_gamma non-NULL) and then RoPE
 * (coords non-NULL) to q and k, in the order of
 * src/sparse_transformer.cpp:202-224. */
int pxs_qkv_prepare(int dtype, const void * qkv, int64_t rows, int heads, int head_dim,
                    const float * q_gamma, const float * k_gamma, const int32_t * coords,
                    float freq_min, float freq_base, void * q, void * k, void * v,
                    void * stream);

/* In-place activation (PXS_ACT_*) over count elements. */
int pxs_activation(int dtype, void * x, int64_t count, int act, void * stream);

/* ---- a7, a9: varlen attention ---------------------------------------------------- */

/* sparse_scaled_dot_product_attention / sparse_cross_attention
 * (src/sparse.cpp:704-859) as one flash-style kernel: queries of segment s,
 * rows [cu_q[s], cu_q[s+1]), attend to keys/values [cu_k[s], cu_k[s+1]).
 * q, k [*, heads * head_dim], v, o [*, heads * head_dim] with row strides
 * ld_* (elements).  cu_q/cu_k are device int64[nseg + 1]; total_q = cu_q[nseg].
 * row_map (nullable, device int32): logical row i is physical row row_map[i]
 * for q, k, v and o alike (window attention reads the permuted order without
 * moving rows).  head_dim must be 64 for PXS_BF16 (MFMA path) and <= 128 for
 * PXS_F32.  A segment with queries but no keys writes zeros.
 * workspace: pxs_attention_workspace_bytes(nseg). */
size_t pxs_attention_workspace_bytes(int nseg);
int pxs_varlen_attention(int dtype, const void * q, int64_t ld_q, const void * k, int64_t ld_k,
                         const void * v, int64_t ld_v, const int64_t * cu_q,
                         const int64_t * cu_k, int nseg, int64_t total_q,
                         const int32_t * row_map, int heads, int head_dim, float scale, void * o,
                         int64_t ld_o, void * workspace, void * stream);

/* Per-batch cu_seqlens from the batch column (src/sparse.cpp:731-737):
 * cu (device int64[batch_size + 1]). */
int pxs_batch_cu_seqlens(const int32_t * coords, int64_t n, int batch_size, int64_t * cu,
                         void * stream);

/* ---- a8: shifted-window partition ------------------------------------------------ */

/* Window partition (no reference counterpart; contract): window
 * w = floor((xyz + shift) / window) per axis, per-axis counts
 * ceil((S + shift) / window), wid = ((b*nx + wx)*ny + wy)*nz + wz.
 * fwd = stable sort of rows by wid, bwd = its inverse; cu_seqlens
 * (capacity n + 1) bounds the non-empty windows in ascending wid and
 * *nwin_out (device int64) receives their count. */
size_t pxs_window_partition_workspace_bytes(int batch_size, int sx, int sy, int sz, int window,
                                            int shift, int64_t n);
int pxs_window_partition(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                         int sz, int window, int shift, int32_t * fwd, int32_t * bwd,
                         int64_t * cu_seqlens, int64_t * nwin_out, void * workspace,
                         void * stream);

#ifdef __cplusplus
}
#endif

#endif /* PXS_H */
