/* C ABI of libmaloq_hip.so: MI355X (gfx950) kernels for MALOQ's equivariant
 * message-passing hot path.
 *
 * Conventions for every entry point:
 *   - All pointers are device pointers unless stated otherwise; tensors are
 *     row-major and contiguous.
 *   - `stream` is a hipStream_t passed as void*; work is enqueued, never synced.
 *   - Return 0 on success, non-zero on error; maloq_last_error() gives the text.
 *   - fp32 unless a `dtype` argument says otherwise (0 = fp32, 1 = bf16 with
 *     fp32 accumulation).
 *
 * Each declaration names the reference interface (file:line under
 * src/maloq/) it replaces.
 */
#ifndef MALOQ_HIP_H
#define MALOQ_HIP_H

#include <stdint.h>

#define MALOQ_ABI_VERSION 3

#ifdef __cplusplus
extern "C" {
#endif

int maloq_abi_version(void);
const char* maloq_last_error(void);

/* ------------------------------------------------------------ Wigner-D -- */

/* Euler triple (alpha, beta, gamma) per edge, as fed to wigner_D:
 * (-gamma, -beta, -alpha) with gamma = Philox(seed, edge) * 2*pi.
 * edge_vec [E,3] (e3nn y-z-x frame), eulers [E,3].
 * Replaces extract_euler_angles, helm/triton_kernels/wigner_fused.py:383-397
 * (and init_edge_rot_euler_angles, helm/common/rotation.py:68-83). */
int maloq_edge_euler(const float* edge_vec, int64_t num_edges, uint64_t seed, float* eulers,
                     void* stream);

/* Dense block-diagonal Wigner-D [E,d,d], d=(lmax+1)^2, 0<=lmax<=8, built from
 * edge vectors in one launch.  jd_packed: J_0..J_lmax row-major, concatenated.
 * eulers_out (nullable) receives the angles used.  wigner / wigner_inv
 * (either nullable) receive D and D^T.  write_zeros != 0 also stores the
 * off-diagonal zeros (else only diagonal blocks are written).
 * Replaces edge_vec_to_wigner_fused, helm/triton_kernels/wigner_fused.py:403-486,
 * plus the transpose().contiguous() of helm/esen_osh.py:294. */
int maloq_edge_vec_to_wigner(const float* edge_vec, int64_t num_edges, uint64_t seed, int lmax,
                             const float* jd_packed, float* eulers_out, float* wigner,
                             float* wigner_inv, int write_zeros, void* stream);

/* Same, from given Euler triples [E,3].
 * Replaces eulers_to_wigner, helm/common/rotation.py:19-39. */
int maloq_wigner_from_euler(const float* eulers, int64_t num_edges, int lmax,
                            const float* jd_packed, float* wigner, float* wigner_inv,
                            int write_zeros, void* stream);

/* Rotation of irreps rows into or out of the edge frame, per edge:
 *   out[e] = D_e x[g(e)]    (inverse == 0),   out[e] = D_e^T x[g(e)]   (inverse != 0),
 * g(e) = gather[e] (nullable: e), x [*, d, c], out [E, d, c], d = (lmax+1)^2,
 * 0 <= lmax <= 8, c a multiple of 4; x_dtype / out_dtype 0 fp32, 1 bf16 (fp32
 * arithmetic).  D_e from exactly one of eulers [E, 3] (the (alpha, beta, gamma)
 * triple of maloq_edge_euler, with jd_packed; bit-identical blocks to
 * maloq_wigner_from_euler) or wigner [E, d, d] fp32 (its diagonal blocks; the
 * reference's Wigner matrices are zero elsewhere).
 * Replaces torch.bmm(wigner, x_message) / torch.bmm(wigner_inv, x_message),
 * helm/esen_block.py:181,191 and helm/esen_osh.py:1218,1228,1318,1328. */
int maloq_rotate(int x_dtype, int out_dtype, int lmax, const void* x, int c, const int32_t* gather,
                 int64_t num_edges, const float* eulers, const float* wigner, const float* jd_packed,
                 int inverse, void* out, void* stream);

/* ------------------------------------------------------ basis transform -- */

/* CG tables shared by the three transform entry points below.  The transform
 * is block diagonal: CG block b (one shell pair l1 x l2) maps the n = (2l1+1)(2l2+1)
 * columns col0 .. col0+n-1 of an unsorted label row to the same columns of the
 * unsorted irreps row (and back).
 *   blocks [nblocks, 4] = (n, col0, woff, program); the block matrix is
 *     w[woff + j*n + k] (output column j, input column k), n in
 *     {1,3,5,7,9,15,21,25,35,49} (l <= 3); program >= 0 names the compiled CG
 *     program (maloq_basis_cg_block) whose matrix equals that block exactly,
 *     which the kernels then run instead of reading w; -1 for none.  The
 *     program depends on the direction (w_fwd / w_inv / w_adj), so each
 *     direction has its own blocks table;
 *   w      the block matrices; NULL is allowed when every block of the table
 *     has a program (the kernels then carry no dense path at all);
 *   sched  column groups and per-wave block lists.  The unsorted row is split
 *     into ngroups groups of consecutive CG blocks (at most 64 blocks and
 *     group_cols columns each; one group of t columns when the row fits one
 *     LDS tile).  sched[0] = ngroups; sched[1 + 4g .. 4 + 4g] = (first column,
 *     width, first block, offset o_g) of group g; sched[o_g .. o_g + 4] are
 *     offsets into sched + o_g + 5 of the (global) block ids of the group's 4
 *     lists; each wave of a workgroup contracts one list (4 waves) or every
 *     other block of one (8 waves);
 *   t      row width (any; the widest group, group_cols, must fit a 32-row
 *     fp32 LDS tile: group_cols <= 1269);
 *   ngroups, group_cols  as in sched; the grid is (row tiles) x (groups).
 * Sorted irreps rows use perm (sorted column j <-> unsorted column perm[j]),
 * only with ngroups = 1 (rows of several groups are permuted by a separate
 * maloq_gather_columns).  Replaces the label-width-agnostic grid of the
 * reference's Triton backend, basis_transform_triton_backend.py:1255-1438. */

/* Label/irreps rows -> rows, [R, t] -> [R, t]:
 *   out[r, j] = Y[r, perm_out ? perm_out[j] : j],  Y = blockdiag(W) X,
 *   X[r, perm_in ? perm_in[j] : j] = in[r, j].
 * With the host's tables one call implements get_net_out
 * (utils_tensor_decomp.py:163-169), get_H (:154-161) and the get_H backward
 * (basis_transform_triton_backend.py:1064-1073).
 * Replaces BalancedTritonE3TensorDecompL2._get_H_impl/_get_net_out_impl,
 * fock_utils/basis_transform_triton_backend.py:1366-1438 (kernels K6/K8). */
int maloq_label_transform(const float* in, const int32_t* perm_in, float* out,
                          const int32_t* perm_out, int64_t num_rows, int t, int nblocks,
                          const int32_t* blocks, const float* w, const int32_t* sched,
                          int ngroups, int group_cols, void* stream);

/* Row plan of the Fock-side transforms, int4 per atom pair r (i = rows[r],
 * j = cols[r]): (base lo, base hi, r, (kind + 1) | n_i << 16 | n_j << 24), where
 *   dense  (data_offsets == NULL): the block starts at fock[off[i]*ld + off[j]], row stride
 *          ld < 2^23;
 *   sparse (data_offsets != NULL): block r at fock[data_offsets[r]], n_j = off[j+1]-off[j]
 *          columns, row-major (SparseBlockMatrix, matrix2labels_kernels.py:43-48);
 * kind = pair_kind[Z_i*100 + Z_j] (-1: no template, the row is all zero), n_i, n_j <= 255,
 * n_i * n_j <= maxe (the template's largest block).  row_meta: [num_rows, 4] int32,
 * 16-byte aligned.  The transforms below take the plan in any row order; entry p of
 * the plan reads and writes row r = plan[p].z.  Replaces the per-call index lists of
 * cupy_single_matrix2label (matrix2labels_kernels.py:978-994). */
int maloq_basis_row_meta(int64_t ld, const int64_t* data_offsets,
                         const int32_t* fock_block_offsets, const int32_t* atomic_numbers,
                         const int32_t* rows, const int32_t* cols, int64_t num_rows,
                         const int32_t* pair_kind, int maxe, int32_t* row_meta, void* stream);

/* Fused Fock -> irreps over a row plan: gather every atom-pair block into its
 * label row, then get_net_out; out [R, t] in original row order.
 * ld: the dense row stride, 0 for block-list storage (as in the plan).
 * slots: the template's elements per (column group, element-pair kind), as a
 *   rectangle of the atom-pair block: slots[0] = kinds K, slots[1] = ngroups,
 *   slots[2 + g] = the largest rectangle (nr * nc) of group g,
 *   slots[2 + ngroups + g*K + k] = r0 | nr << 8 | c0 << 16 | nc << 24 (block rows
 *   r0 .. r0+nr-1, columns c0 .. c0+nc-1; nr = 0 for none; a rectangle outside a
 *   row's actual block is skipped), slots[2 + ngroups + ngroups*K + g*K + k] = the
 *   offset in slots of its column table: nr*nc entries, row-major, each the
 *   column of group g (label column = the group's first column + it) that the
 *   element goes to, or -1.  Label columns no element reaches are zero.
 * kind_blocks [ngroups*K, 2] (or NULL): bit i set if the kind has the group's
 * i-th CG block; blocks that no row of a tile has are skipped.
 * Replaces cupy_single_matrix2label(forward=True) + get_net_out,
 * fock_utils/matrix2labels_kernels.py:946-1036 (K12) / :1038-1115 (K13) and
 * fock_targets_batched.py:426-441. */
int maloq_fock_to_irreps(const float* fock, int64_t ld, const int32_t* row_meta,
                         int64_t num_rows, const int32_t* slots, int maxe,
                         const uint32_t* kind_blocks, float* out, const int32_t* perm_out,
                         int t, int nblocks, const int32_t* blocks, const float* w,
                         const int32_t* sched, int ngroups, int group_cols, void* stream);

/* Fused irreps -> Fock over a row plan: get_H per row, then scatter the label
 * columns that the row's element pair has into its atom-pair block (tables as
 * above; every Fock entry is written by one (row, column), entries no template
 * covers are left untouched).
 * Replaces get_H + cupy_single_matrix2label(forward=False),
 * train_utils/splittrainer.py:546-597 over matrix2labels_kernels.py:946-1036. */
int maloq_irreps_to_fock(const float* irreps, const int32_t* perm_in, float* fock, int64_t ld,
                         const int32_t* row_meta, int64_t num_rows, const int32_t* slots,
                         int maxe, const uint32_t* kind_blocks, int t, int nblocks,
                         const int32_t* blocks, const float* w, const int32_t* sched,
                         int ngroups, int group_cols, void* stream);

/* The two fused transforms above for a one-off pair list, without a row plan:
 * each workgroup describes its own rows exactly as maloq_basis_row_meta would
 * (the same ld / data_offsets / fock_block_offsets / atomic_numbers / rows /
 * cols / pair_kind / maxe arguments), so a single call does the work of
 * maloq_basis_row_meta + maloq_fock_to_irreps (or maloq_irreps_to_fock) with
 * identical results.  For block-list storage ld is ignored.  Replaces the same
 * reference calls as those two; a caller that transforms one structure once
 * (make_targets per molecule and spin, fock_targets_batched.py:426-441) needs
 * no plan. */
int maloq_fock_to_irreps_pairs(const float* fock, int64_t ld, const int64_t* data_offsets,
                               const int32_t* fock_block_offsets, const int32_t* atomic_numbers,
                               const int32_t* rows, const int32_t* cols, int64_t num_rows,
                               const int32_t* pair_kind, const int32_t* slots, int maxe,
                               const uint32_t* kind_blocks, float* out, const int32_t* perm_out,
                               int t, int nblocks, const int32_t* blocks, const float* w,
                               const int32_t* sched, int ngroups, int group_cols, void* stream);
int maloq_irreps_to_fock_pairs(const float* irreps, const int32_t* perm_in, float* fock, int64_t ld,
                               const int64_t* data_offsets, const int32_t* fock_block_offsets,
                               const int32_t* atomic_numbers, const int32_t* rows, const int32_t* cols,
                               int64_t num_rows, const int32_t* pair_kind, const int32_t* slots,
                               int maxe, const uint32_t* kind_blocks, int t, int nblocks,
                               const int32_t* blocks, const float* w, const int32_t* sched,
                               int ngroups, int group_cols, void* stream);

/* The dense n x n matrix (row-major, output column x input column) of compiled
 * CG program p = dir * 16 + l1 * 4 + l2 (dir 0: get_net_out, the
 * decomposition's wms_H block; 1: get_H, its wms block; 2: get_H's adjoint,
 * wms transposed), n = (2 l1 + 1)(2 l2 + 1), written to host memory w.  No GPU
 * work: the host compares its tables with these to fill the program column of
 * blocks.  The matrices restate e3TensorDecomp's blocks for one shell pair,
 * fock_utils/utils_tensor_decomp.py:85-99. */
int maloq_basis_cg_block(int program, float* w, int n);

/* Plain Fock <-> label copy (no CG), dense or block-sparse storage as above.
 * forward != 0: label[r, out0 + k] = block(r)[r0 + k/w, c0 + k%w];
 * forward == 0: the reverse copy.  Template CSR: tmpl_ptr [100*100+1],
 * tmpl [n, 5] = (r0, r1, c0, c1, out0).
 * Replaces cupy_single_matrix2label / cupy_single_matrix2label_sparse,
 * fock_utils/matrix2labels_kernels.py:946-1115 (kernels K12, K13). */
int maloq_matrix2label(float* fock, int64_t ld, const int64_t* data_offsets,
                       const int32_t* fock_block_offsets, const int32_t* atomic_numbers,
                       const int32_t* rows, const int32_t* cols, int64_t num_rows,
                       const int32_t* tmpl_ptr, const int32_t* tmpl, float* target,
                       int64_t target_ld, int forward, void* stream);

/* ------------------------------------------------ Fock irreps head -- */

/* The gated nonlinearity of Fock_Irreps_Head.process (helm/esen_osh.py:986-1005)
 * on backbone features x [R, d, c] (d = (lmax+1)^2, l-major rows, fp32) and the
 * scalar linear's output scalars [R, c + lmax c]:
 *   out[r, 0, k] = scalars[r, k];
 *   out[r, l^2 + m, k] = cst f(scalars[r, c + (l-1) c + k]) x[r, l^2 + m, k], l >= 1
 * with f = sigmoid (act 0) or, with reduce_edge (gates on |scalars|, tanh, so
 * odd data stay odd: :625-629, 994-995), f(z) = tanh(|z|) (act 1); cst: the
 * normalisation of e3nn's Gate activation.  out [R, d, c].  Replaces lin_scalars'
 * split + Gate (e3nn.nn.Gate) of the reference. */
int maloq_irreps_gate_fwd(const float* x, int64_t num_rows, int lmax, int c, const float* scalars, float cst,
                          int act, float* out, void* stream);

/* Its gradient: grad_x [R, d, c] (row 0 is set to zero: x's l = 0 reaches the
 * output only through the scalar linear) and grad_scalars [R, c + lmax c]. */
int maloq_irreps_gate_bwd(const float* x, int64_t num_rows, int lmax, int c, const float* scalars, float cst,
                          int act, const float* grad_out, float* grad_x, float* grad_scalars, void* stream);

/* out[r, k] = src[k] >= 0 ? sign[k] in[r, src[k]] : 0 for k < t (row strides
 * ld_in, ld_out): the head's output permutation to label order
 * (x_out[:, output_permutation], esen_osh.py:909-914, 948-953), with the parity
 * multipliers as signs expand_reduced_node (:1055-1064), and with reduce_edge the
 * alpha and beta terms of the edge-pair remix (:915-937). */
int maloq_gather_columns(const float* in, int64_t ld_in, int64_t num_rows, const int32_t* src, const float* sign,
                         int t, float* out, int64_t ld_out, void* stream);

/* The gradient of that gather: grad_in[r, s] = sum over k in [ptr[s], ptr[s+1])
 * of sign[k] grad_out[r, cols[k]] (the output columns that read input column s,
 * CSR by input column, summed in a fixed order). */
int maloq_scatter_columns(const float* grad_out, int64_t ld_out, int64_t num_rows, const int32_t* ptr,
                          const int32_t* cols, const float* sign, int s, float* grad_in, int64_t ld_in,
                          void* stream);

/* ------------------------------------------- label-side caller hooks -- */

/* labels[r][cols[k]] += sign * means[atomic_numbers[r]][k] for r < num_rows,
 * k < ncols (labels row stride ld, means [max Z + 1, ncols] fp32, every Z of
 * the rows inside the table).  sign = -1: the l = 0 shift of the node labels,
 * Fock_Targets.scale_shift_node_blocks (fock_utils/fock_targets_batched.py:1093-1115,
 * applied at :444-453); sign = +1: its undo, unscale_shift_node_blocks with
 * shift only (:1157-1183, called from train_utils/splittrainer.py:537-541). */
int maloq_label_scalar_shift(float* labels, int64_t ld, int64_t num_rows, const int32_t* atomic_numbers,
                             const float* means, const int32_t* cols, int ncols, float sign, void* stream);

/* Label padding mask: mask[r][c] = cover[pair_kind[Z[rows[r]]*100 + Z[cols[r]]]][c]
 * (0 where the pair kind is -1), mask [num_rows, t] uint8, cover [kinds, t]
 * uint8 (1 on the output columns of every template entry of the kind), Z < 100.
 * Replaces Fock_Targets.create_label_unpadding_mask,
 * fock_utils/fock_targets_batched.py:1012-1080 (a Python loop per row there). */
int maloq_label_mask(const int32_t* rows, const int32_t* cols, const int32_t* atomic_numbers,
                     const int32_t* pair_kind, const uint8_t* cover, int t, int64_t num_rows, uint8_t* mask,
                     void* stream);

/* out[i][j] = sign[i] sign[j] H[src[i]][src[j]] for i, j < n (src a
 * permutation of 0..n-1, sign +-1; out must not alias H): the per-shell
 * m-reordering with reflections S H S^T of sort_by_m,
 * fock_utils/utils_orca_out.py:402-465, with (src, sign) from the host. */
int maloq_signed_permute(const float* H, int64_t n, int64_t ld_in, const int32_t* src, const float* sign,
                         float* out, int64_t ld_out, void* stream);

/* A SparseBlockMatrix (block b: rows of atom block_rows[b], columns of atom
 * block_cols[b], row-major at data[block_data_offsets[b]]) into CSR arrays:
 * indptr [n + 1] and block_col_offsets [num_blocks] (the columns of the blocks
 * left of b in its block row, blocks of a row atom ordered by column atom)
 * from the host; csr_data / csr_indices [nnz] written here, column indices
 * ascending within each row.  Replaces the COO build of
 * sparse_block_matrix_to_scipy_csr, fock_utils/matrix2labels_kernels.py:16-42. */
int maloq_blocks_to_csr(const float* data, const int64_t* block_data_offsets, const int32_t* block_rows,
                        const int32_t* block_cols, const int32_t* fock_block_offsets,
                        const int64_t* block_col_offsets, const int64_t* indptr, int64_t num_blocks,
                        float* csr_data, int64_t* csr_indices, void* stream);

/* -------------------------------------------------- fused message block -- */

/* Floats of the partial-segment buffer the message entry points need. */
int64_t maloq_message_partials_floats(int lmax, int gate, int64_t num_edges, int c_out);

/* Bytes of the packed weight fragments for a (dtype, lmax, mmax, gate,
 * kernel-input channels c_k, kernel-output channels c_n); -1 if unsupported. */
int64_t maloq_message_wpack_bytes(int dtype, int lmax, int mmax, int gate, int c_k, int c_n);

/* Weight packing: out[i] = W[idx[i]] converted to the operand type (dtype 0 =
 * fp32, 1 = bf16, round to nearest even), W being the concatenation of the nsrc
 * fp32 device arrays srcs[k] of src_sizes[k] elements (fc_m0.weight, then
 * so2_m_conv[m-1].fc.weight for m = 1..mmax, in the reference's layout).  idx
 * [n] int64 device array: the fragment order of the kernels, built once per
 * shape by the host packer (maloq_amd.message._pack_index); n elements make
 * maloq_message_wpack_bytes(...) bytes.  nsrc <= 8.  Stands in for reading
 * fc_m0 / so2_m_conv weights at helm/nn/so2_layers.py:161-203 (the kernels
 * take the weights in fragment order). */
int maloq_message_pack(int dtype, int nsrc, const float* const* srcs, const int64_t* src_sizes,
                       const int64_t* idx, int64_t n, void* out, void* stream);

/* Kept rows d' = (lmax+1) + sum_{m=1..mmax} 2 (lmax-m+1) of the m-major layout,
 * and floats per edge of the kept Wigner-D rows (|m| <= mmax) in the kernels'
 * pair-major layout: per degree l, (l+1) column pairs (j, j+1) of the
 * nq = 1 + 2 min(mmax, l) row types, [q][2] padded to a multiple of 4 floats. */
int maloq_message_kept_rows(int lmax, int mmax);
int maloq_message_wigner_floats(int lmax, int mmax);

/* 1 if the message-block kernels are built for (lmax, mmax), else 0: (2, 2),
 * (4, 2), (4, 4), (6, 2), (6, 6).  The reference builds its models with
 * mmax = lmax (train_utils/training_workflow.py:510-511); mmax = 2 is the
 * benchmark's truncation.  Lets a host layer reject a shape at construction
 * (as SO2_Convolution would build it, helm/nn/so2_layers.py:71-130). */
int maloq_message_supported(int lmax, int mmax);

/* Kept Wigner rows (|m| <= mmax) of a caller's dense wigner [E, d, d] fp32 (the
 * reference's argument, esen_block.py:118-121) in the kernels' pair-major
 * layout: dk [E, maloq_message_wigner_floats(lmax, mmax)], dk[p] from
 * wigner[perm[p]] (perm nullable: p).  With eulers == NULL the message
 * forwards below read their dk_ws as so filled instead of building the rows
 * from Euler angles.  Replaces the row selection of bmm(wigner, x_message) +
 * einsum(to_m), helm/esen_block.py:181-184. */
int maloq_message_wigner_rows(int lmax, int mmax, const float* wigner, const int64_t* perm,
                              int64_t num_edges, float* dk, void* stream);

/* Fused message block, forward:
 *   out[n] = sum_{e: dst[e]=n} D_e^T SO2(D_e x[src[e]] (*) rad[e]) [gate],
 * with D_e the kept rows |m| <= mmax of the Wigner-D of eulers[e] (eulers NULL: of the
 * rows dk_ws already holds, see maloq_message_wigner_rows; likewise for
 * maloq_message_edgewise_fwd).
 * Edges must be sorted by dst (non-decreasing); per-edge arrays (eulers, rad)
 * follow that order.  x [N_src, d, c_in] (fp32 or bf16 per dtype), rad
 * [E, sum_m (lmax-m+1) c_in] (nullable), wpack from the host packer, bias
 * [gate ? lmax*c_out + (lmax+1)*c_out : (lmax+1)*c_out] fp32 (nullable),
 * out [num_nodes, d, c_out] fp32, seg_ptr [num_nodes+1] CSR of dst, partials
 * of maloq_message_partials_floats floats.  Workspaces (also the saved
 * tensors of the backward): y_ws [E, d', c_in] (dtype) receives the rotated,
 * radially scaled SO(2) input rows (m-major), r_ws (nullable, same shape) the
 * unscaled rows, dk_ws [E, maloq_message_wigner_floats] fp32 the kept
 * Wigner-D rows; gate_ws (gated blocks, nullable) [E, d' + lmax, c_out] (dtype)
 * the pre-activation rows (kept rows, then the gate rows of degrees 1..lmax)
 * that the gated backward needs.  Two kernels: a per-edge prep (Wigner rows + rotation) and
 * the SO(2) MFMA GEMM with inverse rotation and segment sum, then a fixup for
 * segments cut by tile boundaries.
 * Replaces Edgewise.forward_node, helm/esen_block.py:146-208 (bmm(wigner),
 * einsum(to_m), SO2_Convolution helm/nn/so2_layers.py:139-214, GateActivation
 * helm/nn/activation.py:57-77, bmm(wigner_inv), index_add_). */
int maloq_message_fwd(int dtype, int lmax, int mmax, int gate, const void* x, int c_in,
                      const int32_t* src, const int32_t* dst, int64_t num_edges,
                      const float* eulers, const void* rad, const void* wpack, const float* bias,
                      const float* jd, float* out, int64_t num_nodes, int c_out,
                      const int64_t* seg_ptr, float* partials, void* y_ws, void* r_ws,
                      float* dk_ws, void* gate_ws, void* stream);

/* Bytes of the device array behind maloq_message_fwd_noalloc (per GPU). */
#define MALOQ_NOALLOC_SCRATCH_BYTES (64ll << 20)

/* maloq_message_fwd without allocation: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * result as maloq_message_fwd minus its workspaces (partials, y_ws, r_ws,
 * dk_ws, gate_ws), which come from one file-scope device array of
 * MALOQ_NOALLOC_SCRATCH_BYTES per GPU; eulers must be given (no dense-wigner
 * rows).  The workspace is partials + E d' c_in s + E WS 4 bytes, each part
 * rounded up to 256 (d' = maloq_message_kept_rows, WS =
 * maloq_message_wigner_floats, s = 2 for bf16, 4 for fp32); a call that needs
 * more is refused with an error (about 10 k edges at lmax 4, mmax 2, C 128,
 * bf16).  Nothing is saved for a backward.  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialised by the caller. */
int maloq_message_fwd_noalloc(int dtype, int lmax, int mmax, int gate, const void* x, int c_in,
                              const int32_t* src, const int32_t* dst, int64_t num_edges,
                              const float* eulers, const void* rad, const void* wpack, const float* bias,
                              const float* jd, float* out, int64_t num_nodes, int c_out,
                              const int64_t* seg_ptr, void* stream);

/* Two-convolution message block (forward, node output), as Edgewise.forward_node
 * with message_type "source-target" (helm/esen_block.py:146-208, convolutions
 * :85-106): per dst-sorted edge e, m_e = cat(x[src[e]], x[dst[e]]) (2 c_x channels),
 *   z_e = Gate(SO2_1(rad[e] (*) to_m D_e m_e))   (c_hidden channels, edge frame),
 *   out[n] = sum_{e: dst[e]=n} D_e^T to_m^T SO2_2(z_e)   (c_out channels),
 * SO2_1 gated (wpack1/bias1 packed as for maloq_message_fwd with gate = 1, input
 * 2 c_x), SO2_2 without radial scale or gate (wpack2/bias2, input c_hidden).
 * Workspaces: y_ws [E, d', 2 c_x], z_ws [E, d', c_hidden] (dtype), dk_ws
 * [E, maloq_message_wigner_floats], partials maloq_message_partials_floats(lmax, 0,
 * E, c_out) floats; gate_ws (nullable) [E, d' + lmax, c_hidden] receives the
 * first convolution's pre-activations, r_ws (nullable) [E, d', 2 c_x] the rotated
 * message rows before the radial scale (both kept for the backward).
 * x_msg (nullable) [*, d, c_x] (dtype) with msg_row [E]: message_type
 * "source-target-message", m_e = cat(x[src[e]], x[dst[e]], x_msg[msg_row[e]]) of
 * 3 c_x channels (conv1 input and the workspaces' 2 c_x become 3 c_x).  c_x a multiple of 8.  seg_id (nullable:
 * dst) is the output row of each edge, non-decreasing, with seg_ptr its CSR over
 * num_nodes rows: seg_id[e] = e with seg_ptr[i] = i gives the per-edge rows of
 * Edgewise.forward_edge (esen_block.py:210-258).  Replaces the forward of
 * Edgewise.forward_node (esen_block.py:146-208). */
int maloq_message_edgewise_fwd(int dtype, int lmax, int mmax, const void* x, int c_x,
                               const int32_t* src, const int32_t* dst, const int32_t* seg_id,
                               int64_t num_edges,
                               const float* eulers, const void* rad, const void* wpack1,
                               const float* bias1, int c_hidden, const void* wpack2,
                               const float* bias2, const float* jd, float* out, int64_t num_nodes,
                               int c_out, const int64_t* seg_ptr, float* partials, void* y_ws,
                               void* r_ws, float* dk_ws, void* gate_ws, void* z_ws,
                               const void* x_msg, const int32_t* msg_row, void* stream);

/* Input and radial-scale gradients of the two-convolution block
 * (maloq_message_edgewise_fwd), from the forward's workspaces:
 *   dz2_ws [E, d', c_x]       = D_e grad_out[dst[e]]          (conv2 output gradient),
 *   dz1_ws [E, d' + lmax, c_hidden] = GateActivation backward of SO2_2^T(dz2) at
 *                               gate_saved (the forward's gate_ws): dL/dpre, then
 *                               dL/dgate (formed in the transposed GEMM's epilogue),
 *   grad_rad[e] = SO2_1^T(dz1_e) (*) r_saved[e]  (r_saved: the unscaled rotated
 *                 message rows [E, d', 2 c_x]; both nullable together with rad),
 *   grad_x_src / grad_x_dst [num_nodes, d, c_x] fp32: D_e^T rad[e] (*) SO2_1^T(dz1_e)
 *                 restricted to the x[src] channels and summed per source, resp. to the
 *                 x[dst] channels and summed per destination; grad_x = their sum.
 * grad_x_msg (nullable; then a "source-target-message" block, whose 2 c_x
 * above read 3 c_x): [E, d, c_x] fp32, per dst-sorted edge position: the
 * gradient of that edge's x_msg row; edge_seg [E] = 0, 1, ..., E - 1.
 * grad_row (nullable: dst) is the row of grad_out of each edge (e for the
 * per-edge output of forward_edge, grad_out then [E, d, c_x]).
 * Edges in the forward's dst-sorted order (dst, seg_ptr); src_sorted / edge_idx /
 * seg_ptr_src: the same edges sorted by source, edge_idx the dst-sorted position
 * of each.  wpack1_t / wpack2_t: the two convolutions packed for the transposed
 * GEMM (conv1 gated).  c_x a multiple of 32.  partials: maloq_message_partials_floats(lmax,
 * 1, E, c_x) floats.  dz2_ws and dz1_ws feed
 * maloq_message_dw (conv2: dz2 with the forward's z_ws; conv1: dz1 with y_ws).
 * Replaces the autograd backward of Edgewise.forward_node (esen_block.py:146-208). */
int maloq_message_edgewise_bwd_dx(int dtype, int lmax, int mmax, const float* grad_out, int c_x,
                                  const int32_t* dst, const int32_t* grad_row,
                                  const int32_t* src_sorted,
                                  const int32_t* edge_idx, int64_t num_edges, const float* dk,
                                  const void* rad, void* grad_rad, const void* r_saved,
                                  const void* gate_saved, const void* wpack1_t, int c_hidden,
                                  const void* wpack2_t, const float* jd, float* grad_x_src,
                                  float* grad_x_dst, int64_t num_nodes, const int64_t* seg_ptr,
                                  const int64_t* seg_ptr_src, float* partials, void* dz2_ws,
                                  void* dz1_ws, const int32_t* edge_seg,
                                  float* grad_x_msg, void* stream);

/* Input and radial-scale gradients of the fused block:
 *   grad_x[n] = sum_{e: src[e]=n} D_e^T rad[e] (*) SO2^T(G_e),
 *   grad_rad[e] = SO2^T(G_e) (*) R_e   (R_e = D_e x[src[e]]),
 * with G_e = D_e grad_out[dst[e]] (ungated), or for gate != 0 the gradient
 * through GateActivation at the pre-activations gate_saved (the forward's
 * gate_ws): then G_e has d' + lmax rows (the last lmax: dL/dgate), the SO(2)
 * transpose includes the gate weights, and dz_ws has d' + lmax rows per edge.
 * Edges in src-sorted order: src_sorted non-decreasing, dst_by_src the
 * matching dst, edge_idx the forward (dst-sorted) position of each edge,
 * which indexes dk (forward dk_ws), rad, grad_rad, r_saved (forward r_ws) and
 * dz_ws.  wpack_t: weights packed for the transposed GEMM.  dz_ws [E, d',
 * c_out] (dtype) receives the rotated output-gradient rows (for the weight
 * gradient).  dst_sorted (nullable): dst of each edge in the forward
 * (dst-sorted) order; given, those rows are formed in that order, so that the
 * ~E/N consecutive edges of one node read its grad_out rows from cache (the
 * same values as without it).
 * Replaces the autograd backward of Edgewise.forward_node (esen_block.py:146-208). */
int maloq_message_bwd_dx(int dtype, int lmax, int mmax, int gate, const float* grad_out,
                         int c_out, const int32_t* dst_by_src, const int32_t* src_sorted,
                         const int32_t* edge_idx, int64_t num_edges, const float* dk,
                         const void* rad, void* grad_rad, const void* r_saved,
                         const void* wpack_t, const float* jd, float* grad_x, int64_t num_nodes,
                         int c_in, const int64_t* seg_ptr_src, float* partials, void* dz_ws,
                         const void* gate_saved, const int32_t* dst_sorted, void* stream);

/* Rows to allocate for the saved SO(2) rows (y_ws of maloq_message_fwd, dz_ws of
 * maloq_message_bwd_dx) so that maloq_message_dw can read them in whole 128-edge
 * chunks: round_up(num_edges, 128) + 1.  Rows num_edges and up must be zero
 * (the bf16 weight gradient reads them). */
int64_t maloq_message_edge_rows(int64_t num_edges);

/* Floats of the split-K partials buffer of maloq_message_dw. */
int64_t maloq_message_dw_partials_floats(int lmax, int mmax, int gate, int c_out, int c_in,
                                         int splits);

/* Weight gradients of the SO(2) linear from the saved rows:
 *   dW_0 = sum_e dZ_0(e)^T Y_0(e);  for m >= 1 with C_m = sum_e dZ_m^T Y_m over
 *   the stacked (+m, -m) rows: dWr = C[+,+] + C[-,-], dWi = C[-,+] - C[+,-],
 *   dW_m = [dWr; dWi] in the layout of so2_m_conv[m-1].fc.weight.
 * For a gated block (gate != 0) dz has d' + lmax rows per edge (the last lmax:
 * dL/dgate) and dW_0 also holds the gate rows, first: [lmax c_out + (lmax+1) c_out,
 * (lmax+1) c_in], the gate block being sum_e dG(e)^T Y_0(e).
 * dz [E, d', c_out], y [E, d', c_in] (dtype; for bf16 with maloq_message_edge_rows(E)
 * rows, zero from row E on, channels multiples of 8), dw0 [(lmax+1) c_out, (lmax+1) c_in],
 * dwm: host array of mmax device pointers (mmax <= 6), dwm[m - 1] = dW_m
 * [2 (lmax-m+1) c_out, (lmax-m+1) c_in] fp32.  Split-K over edges,
 * partials summed in split order (deterministic).
 * Replaces the autograd weight gradient of SO2_Convolution
 * (helm/nn/so2_layers.py:139-214, SO2_m_Conv :61-67). */
int maloq_message_dw(int dtype, int lmax, int mmax, int gate, const void* dz, const void* y,
                     int64_t num_edges, int c_out, int c_in, int splits, float* partials,
                     float* dw0, float* const* dwm, void* stream);

/* Bias gradient of fc_m0: out[r c + k] = sum_{e < num_edges} rows[e][row0 + r][k]
 * for r < nrows, k < c, where rows [num_edges, rows_per_edge, c] (dtype 0 =
 * fp32, 1 = bf16; c a multiple of 4 resp. 8) are the saved dL/dz rows of
 * maloq_message_bwd_dx.  db0 of fc_m0 is rows [0, lmax+1) (and, gated, the
 * gate bias rows [d', d'+lmax)).  A fixed-order tree over 64-edge blocks:
 * deterministic, fp32 sums.  partials: maloq_message_colsum_partials_floats
 * floats (may be null when that is 0).  Replaces the autograd bias gradient of
 * fc_m0 (helm/nn/so2_layers.py:161-170). */
int64_t maloq_message_colsum_partials_floats(int nrows, int c, int64_t num_edges);
int maloq_message_colsum(int dtype, const void* rows, int rows_per_edge, int row0, int nrows, int c,
                         int64_t num_edges, float* partials, float* out, void* stream);

/* ----------------------------------------------------- edge-degree embedding -- */

/* EdgeDegreeEmbedding.forward (helm/nn/embedding.py:82-141): with u the
 * RadialMLP output [E, (lmax+1) C] (the m = 0 coefficient of every degree l),
 *   emb_e[l^2 + j][c] = D^l_e[l][j] u_e[l][c]   (j = 0 .. 2l)
 * which is the reference's zero padding + einsum(to_m) + bmm(wigner_inv): only
 * the (l^2 + l)-th column of each block of wigner_inv = D^T meets a non-zero.
 *
 * maloq_edge_m0_rows: rows [E, d] fp32, rows[e][l^2 + j] = D^l_e[l][j] (the m = 0
 * row of each block), from exactly one of wigner_inv [E, d, d] fp32 (the
 * reference's input) or eulers [E, 3] fp32 (the (alpha, beta, gamma) triple
 * of maloq_edge_euler) with jd (packed J_l blocks), computing the m = 0 rows
 * with the dense kernel's recurrence (bit-identical to its D).  lmax 0-6. */
int maloq_edge_m0_rows(int lmax, int64_t num_edges, const float* wigner_inv, const float* eulers,
                       const float* jd, float* rows, void* stream);

/* Node mode (edge_out == NULL): x[dst_e] += emb_e / rescale for every edge, in
 * place, x [num_nodes, d, C]; the embedding is rounded to the dtype of x (as
 * the reference casts it) and multiplied by 1 / rescale (within one rounding
 * of the reference's division); edges are visited per node in the order
 * seg_ptr / perm give (dst-sorted, stable: the order of index_add_), summed in
 * fp32 on top of x and stored once.  Edge mode: edge_out [E, d, C] = emb_e in
 * the dtype of x (no rescale), x untouched.  u_dtype / x_dtype: 0 fp32,
 * 1 bf16; channels 1-256.  Deterministic, no atomics. */
int maloq_edge_degree_embed(int u_dtype, int x_dtype, int lmax, const void* u, int64_t num_edges,
                            int channels, const float* rows, const int64_t* seg_ptr, const int64_t* perm,
                            int64_t num_nodes, float rescale, void* x, void* edge_out, void* stream);

/* Gradient of the embedding with respect to u (the autograd backward of the
 * reference's einsum + bmm + index_add_):
 *   grad_u[e][l C + c] = scale sum_j D^l_e[l][j] grad[row_e][l^2 + j][c],
 * row_e = grad_rows[e] (node mode: the dst of edge e, scale = 1 / rescale) or
 * e (grad_rows NULL: edge mode, scale 1).  grad [*, d, C] (g_dtype 0 fp32,
 * 1 bf16), grad_u [E, (lmax+1) C] fp32, rows from maloq_edge_m0_rows. */
int maloq_edge_degree_embed_bwd(int g_dtype, int lmax, const void* grad, const int64_t* grad_rows,
                                int64_t num_edges, int channels, const float* rows, float scale, float* grad_u,
                                void* stream);

/* ------------------------------------------------------------ RadialMLP -- */

/* The radial function of SO2_Convolution: RadialMLP(channels_list)
 * (helm/nn/radial.py:115-142, called at helm/nn/so2_layers.py:152-154), i.e.
 *   u_0 = x;  u_i = SiLU(LayerNorm_i(W_i u_{i-1} + b_i)), i = 1..nhidden;
 *   out = W_o u_H + b_o.
 * widths[nhidden + 2] = channels_list: c_0 (multiple of 4, <= 128), hidden
 * widths (multiples of 32, <= 128), c_out (multiple of 64).  Hidden-layer
 * parameters are host arrays of nhidden device pointers (fp32, 16-byte aligned):
 * weight[i] [c_{i+1}, c_i], bias[i], ln_weight[i], ln_bias[i] [c_{i+1}];
 * eps is LayerNorm's.  out_weight [c_out, c_H], out_bias [c_out] fp32.
 * dtype 0 = fp32, 1 = bf16: the output dtype and the output layer's MFMA
 * operand type (fp32 accumulation); hidden layers always run in fp32. */

/* Bytes of the packed output-layer weights (both layouts). */
int64_t maloq_radial_pack_bytes(int dtype, int c_out, int c_hidden);

/* Forward.  x [E, c_0] fp32; out [E, c_out] (dtype); wpack: workspace of
 * maloq_radial_pack_bytes (written here, read by maloq_radial_bwd); save:
 * nullable [E, c_H] (dtype), the last hidden activation for the backward.
 * Replaces the forward of RadialMLP.net (torch Linear / LayerNorm / SiLU). */
int maloq_radial_fwd(int dtype, int nhidden, const int* widths, const float* x,
                     int64_t num_edges, const float* const* weight, const float* const* bias,
                     const float* const* ln_weight, const float* const* ln_bias, float eps,
                     const float* out_weight, const float* out_bias, void* wpack, void* out,
                     void* save, void* stream);

/* Floats of the partials workspace of maloq_radial_bwd. */
int64_t maloq_radial_bwd_partials_floats(int dtype, int nhidden, const int* widths,
                                         int64_t num_edges);

/* Backward (num_edges >= 1).  grad [E, c_out] (dtype) = dL/dout; save and
 * wpack as written by maloq_radial_fwd with the same parameters.  Outputs
 * (fp32): grad_x [E, c_0] (nullable), grad_hidden = for each hidden layer in
 * order [dW_i (c_{i+1} x c_i), db_i, dln_weight_i, dln_bias_i],
 * grad_out_weight [c_out, c_H], grad_out_bias [c_out].  Per-tile and split-K
 * partials are summed in a fixed order (deterministic).
 * Replaces the autograd backward of RadialMLP.net. */
int maloq_radial_bwd(int dtype, int nhidden, const int* widths, const float* x,
                     int64_t num_edges, const float* const* weight, const float* const* bias,
                     const float* const* ln_weight, const float* const* ln_bias, float eps,
                     const void* wpack, const void* grad, const void* save, float* grad_x,
                     float* partials, float* grad_hidden, float* grad_out_weight,
                     float* grad_out_bias, void* stream);

/* ------------------------------------------------------- segment scatter -- */

/* out[n, :] = sum_{p in [seg_ptr[n], seg_ptr[n+1])} msg[perm ? perm[p] : p, :],
 * summed in p order (deterministic).  msg [E, width], out [N, width].
 * Replaces index_add_, helm/esen_block.py:194-206 and helm/nn/embedding.py:129-131. */
int maloq_segment_sum(const float* msg, const int64_t* perm, const int64_t* seg_ptr,
                      int64_t num_segments, int64_t width, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MALOQ_HIP_H */
