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
 *     the matching *_workspace_bytes query, 256-byte aligned (as hipMalloc
 *     returns; a misaligned one is an argument error).  (A pack's first
 *     upload allocates its 32 MiB of pinned host staging, freed by
 *     pxs_pack_close.)
 *   - Coordinates are int32 rows (batch, x, y, z), read as 16-byte rows, so
 *     a coordinate array starts 16-byte aligned (as any [rows, 4] int32
 *     allocation does).  Features are row-major [rows, channels].
 *     PXS_BF16 data is stored as raw bfloat16 bit patterns (uint16);
 *     arithmetic accumulates in fp32.
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

/* *status = INT64_MAX (no error yet), for calls that min-reduce into it. */
int pxs_status_reset(int64_t * status, void * stream);

/* Min-reduce into *status row * 8 + 7 for the first row of x ([rows,
 * channels], row stride ld) holding a non-finite value: the reference's
 * feature check (src/sparse.cpp:326-331) on a device buffer. */
int pxs_check_finite(int dtype, const void * x, int64_t rows, int channels, int64_t ld,
                     int64_t * status, void * stream);

/* Summary of count fp32 device values, the figures the flow sampler's
 * PIXAL3D_FLOW_NONFINITE_TRACE line prints (trace_features,
 * src/flow_sampler.cpp:25-83): how many values are non-finite, the first
 * one's index (count when none) and value, and min, max, max |v| and the sum
 * over the finite values (+inf, -inf, 0 and 0 when none is finite).  The sum
 * is accumulated in double in a fixed tree order (the reference sums serially
 * in long double).  stats points to device memory. */
typedef struct pxs_value_stats {
    int64_t nonfinite;
    int64_t first_bad;
    double sum;
    float first_bad_value;
    float min;
    float max;
    float max_abs;
} pxs_value_stats;
size_t pxs_value_stats_workspace_bytes(int64_t count);
int pxs_value_stats_f32(const float * x, int64_t count, pxs_value_stats * stats, void * workspace,
                        void * stream);

/* Dense 3x3x3 neighbor map (src/slat_decoder.cpp:609-668): nbr[k * n + p] is
 * the row of voxel (b, x+kd-1, y+kh-1, z+kw-1), k = kd*9 + kh*3 + kw, or n
 * when absent.  masks (nullable) receives bit k set when offset k is present. */
int pxs_neighbor_map_k3(const int32_t * coords, int64_t n, const void * table, int32_t * nbr,
                        uint32_t * masks, void * stream);

/* The same map from a locality-preserving table (the extent-free
 * alternative to the voxel grid): a hash of 4x4x4 bricks, each owning 64
 * entries of a pool that hold the smallest row at each voxel, so a row's 27
 * neighbours come from the few bricks (3.4 on average) its window touches
 * instead of 27 unrelated hash lines.  pxs_voxel_bricks_bytes(n) bytes
 * (16-byte aligned): the hash of the voxel-hash size plus 256 bytes per row
 * for the worst case of one brick per row.  Outputs identical to
 * pxs_voxel_hash_build + pxs_neighbor_map_k3 (the same map the reference
 * builds per convolution, src/slat_decoder.cpp:609-668). */
size_t pxs_voxel_bricks_bytes(int64_t n);
int pxs_voxel_bricks_build(const int32_t * coords, int64_t n, void * table, void * stream);
int pxs_neighbor_map_k3_bricks(const int32_t * coords, int64_t n, const void * table, int32_t * nbr,
                               uint32_t * masks, void * stream);

/* Dense voxel grid: one int32 cell per (b, x, y, z) of the extents
 * [batch_size, sx, sy, sz] (batch_size * sx * sy * sz * 4 bytes; 0 when the
 * extents are invalid) holding the smallest row with that coordinate.  Rows
 * outside the extents are left out.  Where the grid fits comfortably in HBM
 * (17 MB for two 128^3 items) it replaces the hash for neighbour maps: one
 * load per neighbour and no probe chains. */
size_t pxs_voxel_grid_bytes(int batch_size, int sx, int sy, int sz);
int pxs_voxel_grid_build(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                         int sz, void * grid, void * stream);

/* pxs_neighbor_map_k3 over a dense voxel grid of the same coords and
 * extents: identical nbr and masks. */
int pxs_neighbor_map_k3_grid(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                             int sz, const void * grid, int32_t * nbr, uint32_t * masks,
                             void * stream);

/* Generation-tagged voxel grid: one 32-bit cell per (b, x, y, z) of the
 * extents (pxs_voxel_grid_bytes), holding 255 - generation in its top 8 bits
 * and a row (below 2^24) in its low 24.  After a reset (all ones) each insert
 * takes a generation in 1..255 larger than any used since that reset, and
 * lookups with that generation see only its rows, so the grid is refilled
 * once per 255 builds, not per build: a build costs O(rows) instead of
 * O(cells).  Within a generation the smallest row of a coordinate wins, as in
 * pxs_voxel_grid_build.  Generations outside 1..255 and more than 2^24 - 1
 * rows are rejected.  A replacement, for hot loops that rebuild maps over
 * fixed extents, of the per-build std::unordered_map of
 * src/slat_decoder.cpp:630-635. */
size_t pxs_voxel_grid_tagged_bytes(int batch_size, int sx, int sy, int sz);
int pxs_voxel_grid_tagged_reset(void * grid, int batch_size, int sx, int sy, int sz,
                                void * stream);
int pxs_voxel_grid_tagged_insert(const int32_t * coords, int64_t n, int batch_size, int sx,
                                 int sy, int sz, void * grid, uint32_t generation, void * stream);

/* pxs_neighbor_map_k3 over a tagged grid built with the same coords and
 * generation: identical nbr and masks (src/slat_decoder.cpp:609-668). */
int pxs_neighbor_map_k3_grid_tagged(const int32_t * coords, int64_t n, int batch_size, int sx,
                                    int sy, int sz, const void * grid, uint32_t generation,
                                    int32_t * nbr, uint32_t * masks, void * stream);

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

/* sparse_submanifold_conv3d (src/sparse.cpp:999-1055) as pxs_subm_conv3d,
 * with the neighbours looked up in a dense voxel grid of the same coords and
 * extents inside the convolution (each tile reads the 27 cells around its
 * rows' coordinates), so no neighbour map is built or read: the map of
 * src/slat_decoder.cpp:609-668 fused into the gather.  grid is a
 * plain grid (pxs_voxel_grid_build, generation 0) or a tagged one
 * (pxs_voxel_grid_tagged_insert or pxs_map_s2_topology_tagged with that
 * generation, 1..255, at most 2^24 - 1 rows).  Output identical to
 * pxs_subm_conv3d over the grid's map. */
int pxs_subm_conv3d_grid(int dtype, const void * x, const int32_t * coords, int64_t n, int cin,
                         const void * weight, const float * bias, int cout, int batch_size,
                         int sx, int sy, int sz, const void * grid, uint32_t generation, void * y,
                         void * stream);

/* ---- a4, a15: factor-f topology, strided conv, mean downsample ------------- */

/* Workspace of pxs_downsample_topology / pxs_downsample_s2_topology (factor 2)
 * for n rows. */
size_t pxs_downsample_workspace_bytes(int64_t n, int batch_size, int sx, int sy, int sz,
                                      int factor);

/* Output topology of a factor-2 reduction: the unique (b, x/2, y/2, z/2) in
 * lexicographic order (the coordinates sparse_downsample_mean emits,
 * src/sparse.cpp:553-593).  out_coords holds up to n rows; child_map is
 * [8][n] (offset-major, leading dimension n): child c = (x&1) + 2(y&1) +
 * 4(z&1) of output q is input row child_map[c * n + q], or -1.  *m_out
 * (device int64) receives the output row count. */
int pxs_downsample_s2_topology(const int32_t * coords, int64_t n, int batch_size, int sx,
                               int sy, int sz, int32_t * out_coords, int32_t * child_map,
                               int64_t * m_out, void * workspace, void * stream);

/* pxs_downsample_s2_topology for a pipeline that keeps a tagged fine grid:
 * the same out_coords, *m_out and child map (leading dimension ld_map >= n,
 * all 8 slots of the m outputs written, -1 when absent), with the children
 * read from fine_grid (coords inserted with fine_generation), and the whole
 * dense coarse grid written: coarse_grid (pxs_voxel_grid_bytes of the extents
 * ceil(s/2)) ends holding each output row at its cell and INT_MAX elsewhere,
 * ready for pxs_neighbor_map_k3_grid over out_coords with no build of its
 * own.  Three launches: occupancy bits, a blocked scan of their counts, one
 * thread per coarse cell emitting in lexicographic order.  The workspace
 * (pxs_downsample_s2_tagged_workspace_bytes) carries the occupancy bitmap,
 * which must be zero before the first call
 * (pxs_downsample_s2_tagged_workspace_reset) and which every call leaves zero. */
size_t pxs_downsample_s2_tagged_workspace_bytes(int batch_size, int sx, int sy, int sz);

int pxs_downsample_s2_tagged_workspace_reset(void * workspace, int batch_size, int sx, int sy,
                                             int sz, void * stream);
int pxs_downsample_s2_topology_tagged(const int32_t * coords, int64_t n, int batch_size, int sx,
                                      int sy, int sz, const void * fine_grid,
                                      uint32_t fine_generation, int32_t * out_coords,
                                      int32_t * child_map, int64_t ld_map, int64_t * m_out,
                                      void * coarse_grid, void * workspace, void * stream);
/* One level of a U-Net's topology in three launches: pxs_voxel_grid_tagged_insert
 * of coords under generation (which also marks each row's stride-2 cell in
 * the occupancy bitmap of s2_workspace), pxs_neighbor_map_k3_grid_tagged (nbr,
 * masks; its launch also scans the bitmap) and the emit of
 * pxs_downsample_s2_topology_tagged (out_coords, child_map, *m_out,
 * coarse_grid).  Outputs identical to those three calls; the same limits.
 * nbr and masks may both be NULL: the map is then not built (for a consumer
 * that reads the grid itself, pxs_subm_conv3d_grid). */
int pxs_map_s2_topology_tagged(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                               int sz, void * grid, uint32_t generation, int32_t * nbr,
                               uint32_t * masks, int32_t * out_coords, int32_t * child_map,
                               int64_t ld_map, int64_t * m_out, void * coarse_grid,
                               void * s2_workspace, void * stream);

/* The same level split so that its emit rides on the level's first
 * convolution (the reference builds this topology inside sparse_downsample
 * and the strided conv's gather, src/sparse.cpp:553-597 and 682-686, and the
 * neighbour map inside sparse_submanifold_conv3d, src/sparse.cpp:999-1055):
 *   pxs_s2_tagged_insert: the rows into the tagged grid under generation,
 *     each row's stride-2 cell marked in bitmap (generation & 1) of a pair in
 *     s2_workspace (a region of its own); the emit of generation g clears
 *     the other bitmap, so successive builds on one workspace use successive
 *     generations, and pxs_downsample_s2_tagged_workspace_reset precedes the
 *     first and every restart of the generations (as for the grid);
 *   pxs_subm_conv3d_grid_s2_emit: pxs_subm_conv3d_grid over that grid, with
 *     the emit (out_coords, child_map, *m_out, coarse_grid, as
 *     pxs_map_s2_topology_tagged writes them) done by extra workgroups of the
 *     same launch on the bf16 16-byte path, or by a launch after it;
 *   pxs_s2_tagged_emit: the emit alone (n = the fine row count, for the
 *     child map stride check).
 * Outputs identical to pxs_map_s2_topology_tagged without a map followed by
 * pxs_subm_conv3d_grid; the same limits. */
int pxs_s2_tagged_insert(const int32_t * coords, int64_t n, int batch_size, int sx, int sy, int sz,
                         void * grid, uint32_t generation, void * s2_workspace, void * stream);
int pxs_subm_conv3d_grid_s2_emit(int dtype, const void * x, const int32_t * coords, int64_t n,
                                 int cin, const void * weight, const float * bias, int cout,
                                 int batch_size, int sx, int sy, int sz, const void * grid,
                                 uint32_t generation, void * y, int32_t * out_coords,
                                 int32_t * child_map, int64_t ld_map, int64_t * m_out,
                                 void * coarse_grid, void * s2_workspace, void * stream);
int pxs_s2_tagged_emit(int64_t n, int batch_size, int sx, int sy, int sz, const void * grid,
                       uint32_t generation, int32_t * out_coords, int32_t * child_map,
                       int64_t ld_map, int64_t * m_out, void * coarse_grid, void * s2_workspace,
                       void * stream);

/* A U-Net encoder level after pxs_s2_tagged_insert, in one launch: the
 * SubMConv3d of pxs_subm_conv3d_grid_s2_emit (x -> y_a, weights w_a
 * [27, cout_a, cin]) with its stride-2 emit, then the strided conv of
 * pxs_sparse_conv3d_s2 (y_a -> y_b, weights w_b [8, cout_b, cout_a]) over the
 * child map the emit writes.  The reference runs these as
 * sparse_submanifold_conv3d (src/sparse.cpp:999-1055) and a strided conv over
 * the sparse_downsample topology (src/sparse.cpp:553-597, 682-686).  Each
 * strided-conv tile waits, inside the launch, only for the emit and the
 * SubMConv3d tiles that write its inputs, so it runs in the slots the
 * SubMConv3d's last round leaves free.  m is the coarse row count (known on
 * the host from an earlier build of these coordinates; y_b holds m rows); the
 * emit still writes it to *m_out.  bf16 with 65..128 SubMConv3d outputs,
 * more than 64 strided outputs and inputs of other than a multiple of 64
 * channels run chained; other shapes (the SubMConv3d then on neighbourhood
 * ranges) and fp32 run the two calls in sequence.  Outputs identical to pxs_subm_conv3d_grid_s2_emit
 * then pxs_sparse_conv3d_s2.  The waits are bounded: one that gives up (after
 * about a second, which a correct launch never needs) sets an error word,
 * read back (to host or device memory) by pxs_unet_s2_level_error; its
 * launch's results are void.  The word is cleared by
 * pxs_downsample_s2_tagged_workspace_reset. */
int pxs_unet_s2_level(int dtype, const void * x, const int32_t * coords, int64_t n, int cin,
                      const void * w_a, const float * b_a, int cout_a, int batch_size, int sx,
                      int sy, int sz, const void * grid, uint32_t generation, void * y_a,
                      const void * w_b, const float * b_b, int cout_b, int64_t m, void * y_b,
                      int32_t * out_coords, int32_t * child_map, int64_t ld_map, int64_t * m_out,
                      void * coarse_grid, void * s2_workspace, void * stream);
int pxs_unet_s2_level_error(const void * s2_workspace, int batch_size, int sx, int sy, int sz,
                            uint32_t * error_out, void * stream);

/* The same topology for any factor f, as groups: output q (coordinates
 * (b, x/f, y/f, z/f), lexicographic) gathers input rows
 * group_rows[group_offsets[q] .. group_offsets[q+1]) in ascending order.
 * out_coords holds up to n rows, group_offsets n + 1 entries, group_rows n. */
int pxs_downsample_topology(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                            int sz, int factor, int32_t * out_coords, int64_t * group_offsets,
                            int32_t * group_rows, int64_t * m_out, void * workspace,
                            void * stream);

/* Stride-2 SparseConv3d with a 2x2x2 kernel (no reference counterpart; the
 * contract is documented with the topology above): y[q] = sum over present
 * children c of W_c x[child] + bias, weight [8, cout, cin].  ld_map is the
 * leading dimension of child_map (the n passed to the topology call), m the
 * output rows. */
int pxs_sparse_conv3d_s2(int dtype, const void * x, int64_t n_in, int cin, const void * weight,
                         const float * bias, int cout, const int32_t * child_map, int64_t ld_map,
                         int64_t m, void * y, void * stream);

/* sparse_downsample_mean features (src/sparse.cpp:536-602): each output is
 * the sum of its group's rows in ascending row order divided by the count. */
int pxs_downsample_mean(int dtype, const void * x, int channels, const int64_t * group_offsets,
                        const int32_t * group_rows, int64_t m, void * y, void * stream);

/* ---- a5: channel to spatial ---------------------------------------------------- */

/* sparse_channel_to_spatial (src/sparse.cpp:604-702) for factor f (cc = f^3
 * children): x [n, cc * c_out]; subdivision (nullable, fp32 [n, cc]) selects
 * children > 0.  Child c lands at (f x + c % f, f y + (c / f) % f,
 * f z + c / f^2).  Output rows are parent-major, child ascending; out_coords
 * and y hold up to n * cc rows; *m_out (device int64) receives the count. */
size_t pxs_channel_to_spatial_workspace_bytes(int64_t n, int factor);
int pxs_channel_to_spatial(int dtype, const int32_t * coords, int64_t n, const void * x,
                           int channels, int factor, const float * subdivision,
                           int32_t * out_coords, void * y, int64_t * m_out, void * workspace,
                           void * stream);

/* ---- a6: sparse linear --------------------------------------------------------- */

/* sparse_linear / varlen_linear (src/sparse.cpp:337-488): y = x W^T + bias,
 * weight [cout, cin] row-major, then an optional activation (PXS_ACT_*,
 * the GELU-tanh of src/sparse_transformer.cpp:123-134 or the SiLU of
 * src/slat_decoder.cpp:68-78).  bias may be NULL. */
int pxs_linear(int dtype, const void * x, int64_t rows, int cin, const void * weight,
               const float * bias, int cout, int act, void * y, void * stream);

/* fp32 sparse_linear in the reference's own operation order (bias, then
 * inputs ascending, each product and sum rounded alone): bit-equal to
 * src/sparse.cpp:436-446.  One thread per output value, so meant for few
 * outputs where exact signs matter: the decoder's subdivision logits
 * (to_subdiv, 8 outputs), whose sign decides the next level's topology. */
int pxs_linear_ordered(const float * x, int64_t rows, int cin, const float * weight,
                       const float * bias, int cout, float * y, void * stream);

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

/* Linear whose epilogue adds into an fp32 residual: residual[r, o] +=
 * (x W^T + bias)[r, o] (add_in_place, src/sparse_transformer.cpp:57-69). */
int pxs_linear_residual(int dtype, const void * x, int64_t rows, int cin, const void * weight,
                        const float * bias, int cout, float * residual, void * stream);

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

/* y = x converted between PXS_F32 and PXS_BF16 (round to nearest even). */
int pxs_convert(int src_dtype, const void * x, int64_t count, int dst_dtype, void * y,
                void * stream);

/* timestep_embedding (src/flow.cpp:92-123): out [batch, dim] fp32 from
 * timesteps (device fp32 [batch]). */
int pxs_timestep_embedding(const float * timesteps, int64_t batch, int dim, int max_period,
                           float * out, void * stream);

/* ---- a7, a9: varlen attention ---------------------------------------------------- */

/* sparse_scaled_dot_product_attention / sparse_cross_attention
 * (src/sparse.cpp:704-859) as one flash-style kernel: queries of segment s,
 * rows [cu_q[s], cu_q[s+1]), attend to keys/values [cu_k[s], cu_k[s+1]).
 * q, k [*, heads * head_dim], v, o [*, heads * head_dim] with row strides
 * ld_* (elements).  cu_q/cu_k are device int64[nseg + 1]; total_q = cu_q[nseg].
 * row_map (nullable, device int32): logical row i is physical row row_map[i]
 * for q, k, v and o alike (window attention reads the permuted order without
 * moving rows).  head_dim and value_dim (the per-head width of v and o) are
 * 1..512; head_dim == value_dim == 64 in PXS_BF16 takes the fastest kernel,
 * dims up to 64 the tiled MFMA kernels, wider heads a wavefront-per-query
 * kernel (one online-softmax pass over the keys, no head-size limit below 512).
 * A segment with queries but no keys writes zeros.
 * workspace: pxs_attention_workspace_bytes(nseg). */
size_t pxs_attention_workspace_bytes(int nseg);
int pxs_varlen_attention(int dtype, const void * q, int64_t ld_q, const void * k, int64_t ld_k,
                         const void * v, int64_t ld_v, const int64_t * cu_q,
                         const int64_t * cu_k, int nseg, int64_t total_q,
                         const int32_t * row_map, int heads, int head_dim, int value_dim,
                         float scale, void * o, int64_t ld_o, void * workspace, void * stream);

/* pxs_varlen_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * Its scratch (segment tile counts and their prefix sums) lives in a 1 MiB
 * array in the library's device image, one per GPU, held until the process
 * ends; nseg is limited to PXS_ATTN_NOALLOC_MAX_SEGMENTS (a larger count is
 * an argument error).  It allocates nothing and otherwise behaves exactly as
 * pxs_varlen_attention (same kernels, same results).  All calls on one GPU
 * share that array: calls that overlap on one GPU (several streams or host
 * threads) race and must be ordered by the caller. */
#define PXS_ATTN_NOALLOC_MAX_SEGMENTS 65536
int pxs_varlen_attention_noalloc(int dtype, const void * q, int64_t ld_q, const void * k,
                                 int64_t ld_k, const void * v, int64_t ld_v, const int64_t * cu_q,
                                 const int64_t * cu_k, int nseg, int64_t total_q,
                                 const int32_t * row_map, int heads, int head_dim, int value_dim,
                                 float scale, void * o, int64_t ld_o, void * stream);

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
 * *nwin_out (device int64) receives their count.  Entries nwin .. cap, with
 * cap = min(n, batch_size * nx * ny * nz) known on the host, hold n: passing
 * nseg = cap to pxs_varlen_attention (empty trailing segments) needs no read
 * of *nwin_out. */
size_t pxs_window_partition_workspace_bytes(int batch_size, int sx, int sy, int sz, int window,
                                            int shift, int64_t n);
int pxs_window_partition(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                         int sz, int window, int shift, int32_t * fwd, int32_t * bwd,
                         int64_t * cu_seqlens, int64_t * nwin_out, void * workspace,
                         void * stream);

/* ---- a13, a14: transformer block and SLat-flow forward, device resident ----------- */

/* SparseTransformerBlockConfig (include/pixal3d/sparse_transformer.h:13-27). */
typedef struct pxs_block_config {
    int channels;
    int num_heads;
    int mlp_hidden;
    int context_channels;
    int proj_in_channels;
    float norm_eps;
    float rope_freq_min;
    float rope_freq_base;
    int use_rope;
    int qk_rms_norm;
    int qk_rms_norm_cross;
    int use_projection;
} pxs_block_config;

/* SparseTransformerBlockWeightsF32 (include/pixal3d/sparse_transformer.h:29-53),
 * as device pointers in the same order.  Linear weights ([out, in]) are in
 * the call's dtype; modulation, biases, norm affines and RMS gammas are fp32.
 * Optional members (RMS gammas, projection) may be NULL when the config does
 * not use them. */
typedef struct pxs_block_weights {
    const float * modulation;
    const void * self_to_qkv_weight;
    const float * self_to_qkv_bias;
    const float * self_q_gamma;
    const float * self_k_gamma;
    const void * self_to_out_weight;
    const float * self_to_out_bias;
    const float * norm2_weight;
    const float * norm2_bias;
    const void * cross_to_q_weight;
    const float * cross_to_q_bias;
    const void * cross_to_kv_weight;
    const float * cross_to_kv_bias;
    const float * cross_q_gamma;
    const float * cross_k_gamma;
    const void * cross_to_out_weight;
    const float * cross_to_out_bias;
    const void * proj_weight;
    const float * proj_bias;
    const void * mlp0_weight;
    const float * mlp0_bias;
    const void * mlp2_weight;
    const float * mlp2_bias;
} pxs_block_weights;

/* sparse_transformer_cross_block_f32 (src/sparse_transformer.cpp:138-292) on
 * device buffers.  hidden (fp32 [rows, C]) is the residual stream, updated in
 * place; coords [rows, 4] contiguous by batch with per-batch bounds cu_rows
 * (device int64[batch_size + 1]); time_mod fp32 [batch_size, 6C]; context
 * (dtype [context_tokens, context_channels]) with context_offsets (device
 * int64[batch_size + 1]); projected (dtype [rows, proj_in_channels]) only when
 * cfg->use_projection.  Every batch must hold at least one row and one
 * context token (the reference rejects empty key sequences).  GEMM operands
 * are in dtype, accumulation and the residual stream in fp32. */
size_t pxs_transformer_block_workspace_bytes(int dtype, const pxs_block_config * cfg,
                                             int64_t rows, int64_t context_tokens,
                                             int batch_size);
int pxs_transformer_block(int dtype, const pxs_block_config * cfg, const pxs_block_weights * w,
                          const int32_t * coords, int64_t rows, int batch_size,
                          const int64_t * cu_rows, float * hidden, const float * time_mod,
                          const void * context, const int64_t * context_offsets,
                          int64_t context_tokens, const void * projected, void * workspace,
                          void * stream);

/* SLatFlowHParams (include/pixal3d/slat_flow.h:12-36) reduced to what the
 * forward uses; mlp_hidden = model_channels * mlp_ratio. */
typedef struct pxs_flow_config {
    int in_channels;
    int out_channels;
    int model_channels;
    int cond_channels;
    int num_blocks;
    int num_heads;
    int proj_in_channels;
    int mlp_hidden;
    float norm_eps;
    float rope_freq_min;
    float rope_freq_base;
    int qk_rms_norm;
    int qk_rms_norm_cross;
    int use_projection;
} pxs_flow_config;

/* SLatFlowWeightsF32 (include/pixal3d/slat_flow.h:38-50) as device pointers:
 * input, timestep-MLP, adaLN and output layers in fp32; blocks is a host
 * array of num_blocks block weight sets in the call's dtype. */
typedef struct pxs_flow_weights {
    const float * input_weight;
    const float * input_bias;
    const float * timestep_weight0;
    const float * timestep_bias0;
    const float * timestep_weight2;
    const float * timestep_bias2;
    const float * modulation_weight;
    const float * modulation_bias;
    const float * output_weight;
    const float * output_bias;
    const pxs_block_weights * blocks;
} pxs_flow_weights;

/* slat_flow_forward_f32 (src/slat_flow.cpp:161-249): input linear, 256-wide
 * sinusoid -> Linear -> SiLU -> Linear -> SiLU -> adaLN Linear, num_blocks
 * transformer blocks, layer norm (eps 1e-5) and output linear.  x fp32
 * [rows, in_channels], timesteps device fp32 [batch_size], out fp32
 * [rows, out_channels]; context / projected as for pxs_transformer_block. */
size_t pxs_slat_flow_workspace_bytes(int dtype, const pxs_flow_config * cfg, int64_t rows,
                                     int64_t context_tokens, int batch_size);
int pxs_slat_flow_forward(int dtype, const pxs_flow_config * cfg, const pxs_flow_weights * w,
                          const int32_t * coords, int64_t rows, int batch_size,
                          const int64_t * cu_rows, const float * x, const float * timesteps,
                          const void * context, const int64_t * context_offsets,
                          int64_t context_tokens, const void * projected, float * out,
                          void * workspace, void * stream);

/* ---- f4: flow-matching Euler sampler with classifier-free guidance ---------------- */

/* FlowEulerSamplerConfig (include/pixal3d/flow_sampler.h:14-23) without the
 * trajectory flag. */
typedef struct pxs_flow_sampler_config {
    int steps;
    float sigma_min;
    float rescale_t;
    float guidance_strength;
    float guidance_rescale;
    float guidance_interval_min;
    float guidance_interval_max;
} pxs_flow_sampler_config;

/* Host function: the schedule of step `step` of flow_euler_sample_f32
 * (src/flow_sampler.cpp:268-285): the model time t in [0, 1] (the model is
 * called with 1000 t), the next step's t, and the guidance weight (the
 * configured strength inside the guidance interval, else 1).  Rejects the
 * configurations valid_config rejects (src/flow_sampler.cpp:111-124) with its
 * message. */
int pxs_flow_sampler_schedule(const pxs_flow_sampler_config * cfg, int step, float * timestep,
                              float * next_timestep, float * guidance);

/* The guided prediction of one step (src/flow_sampler.cpp:192-235, 304-318):
 * prediction = g * positive + (1 - g) * negative, then, when
 * guidance_rescale > 0, the CFG rescale: x0 = (1 - sigma_min) state -
 * (sigma_min + (1 - sigma_min) t) pred for pred = positive and the blend, the
 * population standard deviation of each batch item's x0 values (rows
 * cu_rows[b] .. cu_rows[b+1]), x0_cfg scaled by std_pos / std_cfg (1 when
 * std_cfg is 0) and mixed with weight guidance_rescale, converted back to a
 * prediction.  All fp32 [rows, channels] device buffers; results equal the
 * reference bit for bit.  coords, cu_rows and the workspace are used by the
 * rescale only.  An item without rows keeps a zero deviation (the reference
 * rejects such input before this step). */
size_t pxs_flow_guidance_workspace_bytes(int batch_size);
int pxs_flow_guidance(const float * state, const float * positive, const float * negative,
                      const int32_t * coords, const int64_t * cu_rows, int64_t rows, int channels,
                      int batch_size, float timestep, float sigma_min, float guidance,
                      float guidance_rescale, float * prediction, void * workspace, void * stream);

/* pred_to_xstart (src/flow_sampler.cpp:138-146): x0 = (1 - sigma_min) state
 * - (sigma_min + (1 - sigma_min) t) prediction, over count fp32 values. */
int pxs_flow_pred_to_xstart(const float * state, const float * prediction, int64_t count,
                            float timestep, float sigma_min, float * x0, void * stream);

/* The Euler step state -= delta * prediction (src/flow_sampler.cpp:330-333),
 * delta = t - t_next. */
int pxs_flow_euler_update(float * state, const float * prediction, int64_t count, float delta,
                          void * stream);

/* flow_euler_sample_f32 (src/flow_sampler.cpp:237-345) with the SLat-flow
 * model of pxs_slat_flow_forward as the velocity, device resident: from
 * noise (fp32 [rows, in_channels]) at t = 1 to samples at t = 0.  Guided
 * steps run the conditional and unconditional forwards as ONE varlen batch
 * of 2 * batch_size items (the rows twice, cond then uncond context), so
 * every launch of the forward carries twice the tokens; a step whose
 * guidance weight is 1 (or 0) runs the conditional (or unconditional)
 * forward alone, as the reference does.  cond / uncond: context tokens in the
 * call's dtype with per-item offsets, as for pxs_slat_flow_forward.  Requires
 * in_channels == out_channels.  samples may alias noise.
 * The reference's finiteness checks run on the device: every step's velocity
 * (check_model_output, src/flow_sampler.cpp:126-136) and, when
 * guidance_rescale > 0, the x0 of the conditional prediction and of the CFG
 * blend (sparse_batch_std, src/flow_sampler.cpp:168).  They collect into one
 * status word that is read after the last step (the call synchronizes
 * `stream` once there); a non-finite value fails the call with PXS_ERR_DATA and
 * the reference's message "sparse features contain a non-finite value", and
 * samples is then undefined (the reference stops at the failing step; the
 * device runs every step and reports at the end). */
size_t pxs_flow_euler_sample_workspace_bytes(int dtype, const pxs_flow_config * cfg,
                                             int64_t rows, int64_t cond_tokens,
                                             int64_t uncond_tokens, int batch_size);
int pxs_flow_euler_sample(int dtype, const pxs_flow_config * cfg, const pxs_flow_weights * w,
                          const pxs_flow_sampler_config * scfg, const int32_t * coords,
                          int64_t rows, int batch_size, const int64_t * cu_rows,
                          const float * noise, const void * cond, const int64_t * cond_offsets,
                          int64_t cond_tokens, const void * uncond,
                          const int64_t * uncond_offsets, int64_t uncond_tokens,
                          float * samples, void * workspace, void * stream);

/* ---- a16: SLat-decoder blocks, device resident ------------------------------------ */

/* SLatDecoderBlockWeightsF32 (include/pixal3d/slat_decoder.h:18-41) as device
 * pointers in the same order.  Convolution weights ([27, out, in]) and the
 * ConvNeXt MLP weights ([out, in]) are in the call's dtype; norms and biases
 * are fp32, and so is to_subdiv_weight (the subdivision logits select
 * children by sign, so they are computed in fp32 in every dtype).  Members a
 * block kind does not use may be NULL. */
typedef struct pxs_decoder_block_weights {
    const float * norm_weight;
    const float * norm_bias;
    const float * norm1_weight;
    const float * norm1_bias;
    const void * conv1_weight;
    const float * conv1_bias;
    const float * norm2_weight;
    const float * norm2_bias;
    const void * conv2_weight;
    const float * conv2_bias;
    const void * mlp0_weight;
    const float * mlp0_bias;
    const void * mlp2_weight;
    const float * mlp2_bias;
    const float * to_subdiv_weight;
    const float * to_subdiv_bias;
} pxs_decoder_block_weights;

/* sparse_convnext_block_f32 (src/slat_decoder.cpp:185-224): y = x +
 * MLP2(SiLU(MLP0(LN_affine(SubMConv3d(x))))) with MLP0 channels -> mlp_hidden.
 * x, y fp32 [rows, channels] and may be the same buffer.  nbr/masks: the
 * level's neighbor map (pxs_neighbor_map_k3), or both NULL to build it in the
 * workspace (have_map = 0 in the size query). */
size_t pxs_convnext_block_workspace_bytes(int dtype, int64_t rows, int channels, int mlp_hidden,
                                          int have_map);
int pxs_convnext_block(int dtype, const int32_t * coords, int64_t rows, const float * x,
                       int channels, int mlp_hidden, float eps,
                       const pxs_decoder_block_weights * w, const int32_t * nbr,
                       const uint32_t * masks, float * y, void * workspace, void * stream);

/* sparse_resblock_c2s_f32 (src/slat_decoder.cpp:226-288): subdivide x
 * [rows, channels] (channels % 8 == 0) to the 2x grid.  Children are selected
 * by subdivision (fp32 [rows, 8], > 0), by the block's own to_subdiv logits
 * when pred_subdiv (written to predicted_subdiv [rows, 8] if non-NULL), or all
 * kept when neither is given.  Output: out_coords [m, 4] and y fp32
 * [m, out_channels] with m <= 8 * rows; *rows_out (host) receives m.  When
 * children are selected the call waits once on the stream to read m.
 * out_channels must be a multiple of channels / 8 (the repeated skip). */
size_t pxs_resblock_c2s_workspace_bytes(int dtype, int64_t rows, int channels,
                                        int out_channels);
int pxs_resblock_c2s(int dtype, const int32_t * coords, int64_t rows, const float * x,
                     int channels, int out_channels, float eps,
                     const pxs_decoder_block_weights * w, int pred_subdiv,
                     const float * subdivision, float * predicted_subdiv, int32_t * out_coords,
                     float * y, int64_t * rows_out, void * workspace, void * stream);

/* One entry of SLatDecoderWeightsF32::blocks (include/pixal3d/slat_decoder.h:
 * 18-41): kind 0 = ConvNeXt, 1 = channel-to-spatial. */
#define PXS_DECODER_CONVNEXT 0
#define PXS_DECODER_C2S 1
typedef struct pxs_decoder_block {
    int kind;
    int channels;
    int out_channels;
    int mlp_hidden;
    pxs_decoder_block_weights w;
} pxs_decoder_block;

/* SLatDecoderConfig (include/pixal3d/slat_decoder.h:46-53); model_channels
 * and num_blocks are host arrays of `levels` entries. */
typedef struct pxs_decoder_config {
    int latent_channels;
    int out_channels;
    float norm_eps;
    int pred_subdiv;
    int levels;
    const int * model_channels;
    const int * num_blocks;
} pxs_decoder_config;

/* slat_decoder_forward_f32 (src/slat_decoder.cpp:290-375) on the device:
 * from_latent linear, then per level num_blocks[l] ConvNeXt blocks (sharing
 * one neighbour map per level) and, except at the last level, the
 * channel-to-spatial block that makes the next level's coordinates; final
 * layer norm (eps 1e-5, no affine) and output linear.  blocks: host array of
 * n_blocks entries in level order.  With upsample_times >= 0 the call is
 * slat_decoder_upsample_coords_f32 (src/slat_decoder.cpp:377-440) instead: it
 * stops after upsample_times C2S levels and returns that level's hidden
 * state (y [m, model_channels[upsample_times]]) with its coordinates.
 * guide (nullable): host array of levels - 1 device fp32 [rows_l, 8]
 * subdivision guides; predicted (nullable, pred_subdiv only): host array of
 * levels - 1 device fp32 buffers of max_rows x 8 that receive each C2S
 * block's logits.  max_rows bounds every level: each C2S needs
 * 8 * rows_l <= max_rows (rows * 8^(levels-1) always suffices).  *rows_out
 * (host) receives the output rows m; level_rows (host, nullable) the rows of
 * each level.  The call waits on the stream once per C2S level to read its
 * row count. */
size_t pxs_slat_decoder_workspace_bytes(int dtype, const pxs_decoder_config * cfg,
                                        const pxs_decoder_block * blocks, int n_blocks,
                                        int64_t rows, int64_t max_rows);
int pxs_slat_decoder_forward(int dtype, const pxs_decoder_config * cfg,
                             const float * from_latent_weight, const float * from_latent_bias,
                             const float * output_weight, const float * output_bias,
                             const pxs_decoder_block * blocks, int n_blocks,
                             const int32_t * coords, int64_t rows, const float * x,
                             const float * const * guide, float * const * predicted,
                             int upsample_times, int64_t max_rows, int32_t * out_coords,
                             float * y, int64_t * rows_out, int64_t * level_rows,
                             void * workspace, void * stream);

/* repeat_channels + add_in_place (src/slat_decoder.cpp:44-107):
 * y[r, j] = a[r, j] + skip[r, j / (channels / skip_channels)], y fp32; a in
 * a_dtype (may be y itself when PXS_F32). */
int pxs_add_repeat(int a_dtype, const void * a, int64_t rows, int channels, const float * skip,
                   int skip_channels, float * y, void * stream);

/* ---- f3: GGUF pack ingestion ------------------------------------------------------- */

/* An open Pixal3D GGUF pack (host object).  The C++ drop-in of the
 * reference reader is include/pixal3d/pack.h. */
typedef struct pxs_pack pxs_pack;

/* load_pack_info + Pixal3DPackReader::open (src/pack.cpp:127-311): parse the
 * GGUF v3 header, metadata and tensor table (no payload) and apply the
 * reference's checks and messages. */
int pxs_pack_open(const char * path, pxs_pack ** pack);
void pxs_pack_close(pxs_pack * pack);

/* Pixal3DPackInfo (include/pixal3d/pack.h:16-47) as a JSON object written to
 * buf (NUL-terminated) when len suffices; returns the length it needs
 * (NUL included), 0 for a NULL pack. */
size_t pxs_pack_describe(const pxs_pack * pack, char * buf, size_t len);

/* Pixal3DPackReader::metadata_* (src/pack.cpp:387-462): the reference's type
 * rules, defaults for a missing optional key (0, 0.0, false, "") and
 * messages. */
int pxs_pack_metadata_u32(const pxs_pack * pack, const char * key, int required,
                          uint32_t * value);
int pxs_pack_metadata_f32(const pxs_pack * pack, const char * key, int required, float * value);
int pxs_pack_metadata_bool(const pxs_pack * pack, const char * key, int required, int * value);
int pxs_pack_metadata_string(const pxs_pack * pack, const char * key, int required, char * buf,
                             size_t len);

/* Pixal3DPackReader::read_tensor (src/pack.cpp:331-385): the payload bytes
 * into host memory dst (capacity bytes); *n_bytes receives the size. */
int pxs_pack_read_tensor(const pxs_pack * pack, const char * name, void * dst, size_t capacity,
                         size_t * n_bytes);

/* Device workspace of the upload calls below (two 16 MiB staging chunks and
 * one flag per tensor of the pack). */
size_t pxs_pack_upload_workspace_bytes(const pxs_pack * pack);

/* read_tensor_f32 (src/slat_flow.cpp:360-395) onto the device: an F32, F16
 * or BF16 tensor converted to dtype (PXS_F32 exactly; PXS_BF16 rounded to
 * nearest even) at dst (device, 16-byte aligned, count = the tensor's
 * elements).  The payload streams file -> pinned staging -> HBM in chunks
 * with the next read overlapping the copy and conversion.  A non-finite
 * value fails with PXS_ERR_DATA.  Waits for `stream`.  Calls on one pack
 * must not overlap (they share its pinned staging). */
int pxs_pack_upload(pxs_pack * pack, const char * name, int dtype, void * dst, int64_t count,
                    void * workspace, void * stream);

/* SLatFlowModel::load (src/slat_flow.cpp:1239-1281) for one component
 * (shape_flow_512, shape_flow_1024, texture_flow_1024): plan reads and checks
 * the hyperparameters (read_hparams / valid_hparams, src/slat_flow.cpp:
 * 397-429, 113-138) into *cfg and sizes the device arena; load converts
 * every tensor of the component into the arena (block linear weights in
 * dtype, everything else fp32, each 256-byte aligned) and binds *w and
 * blocks[0 .. num_blocks) (SLatFlowModel::forward, src/slat_flow.cpp:
 * 1348-1395) for pxs_slat_flow_forward / pxs_flow_euler_sample with the same
 * dtype.  A missing tensor or one whose shape disagrees with the
 * hyperparameters fails the load.  Waits for `stream`. */
int pxs_slat_flow_pack_plan(const pxs_pack * pack, const char * component, int dtype,
                            pxs_flow_config * cfg, size_t * arena_bytes);
int pxs_slat_flow_pack_load(pxs_pack * pack, const char * component, int dtype, void * arena,
                            size_t arena_bytes, void * workspace, pxs_flow_weights * w,
                            pxs_block_weights * blocks, int max_blocks, void * stream);

/* SLatDecoderHParams (include/pixal3d/slat_decoder.h:108-118); n_blocks =
 * sum(num_blocks) + levels - 1 entries of pxs_decoder_block. */
#define PXS_DECODER_MAX_LEVELS 16
typedef struct pxs_decoder_hparams {
    int resolution;
    int latent_channels;
    int out_channels;
    int levels;
    int pred_subdiv;
    int n_blocks;
    float norm_eps;
    int model_channels[PXS_DECODER_MAX_LEVELS];
    int num_blocks[PXS_DECODER_MAX_LEVELS];
} pxs_decoder_hparams;

/* SLatDecoderModel::load (src/slat_decoder.cpp:3392-3467) and make_weights
 * (2911-2970) for one component: plan reads the metadata into *hp and sizes
 * the arena; load converts the component's tensors into the arena
 * (convolution and ConvNeXt MLP weights in dtype, everything else fp32) and
 * fills blocks[0 .. n_blocks) in level order and io_weights[4] =
 * {from_latent weight, bias, output_layer weight, bias} for
 * pxs_slat_decoder_forward (whose config is latent_channels, out_channels,
 * norm_eps, pred_subdiv, levels, model_channels, num_blocks of *hp).  Waits
 * for `stream`. */
int pxs_slat_decoder_pack_plan(const pxs_pack * pack, const char * component, int dtype,
                               pxs_decoder_hparams * hp, size_t * arena_bytes);
int pxs_slat_decoder_pack_load(pxs_pack * pack, const char * component, int dtype, void * arena,
                               size_t arena_bytes, void * workspace, pxs_decoder_block * blocks,
                               int max_blocks, const float ** io_weights, void * stream);

#ifdef __cplusplus
}
#endif

#endif /* PXS_H */
