// Label-side helpers of the Fock <-> irreps path (gfx950): the callers' hooks
// around the basis transform, moved from host loops to the GPU.
//   * l = 0 scale-shift of node labels and its undo
//     (fock_targets_batched.py:444-453, 1093-1115; undo :1157-1194, used at
//     train_utils/splittrainer.py:537-541);
//   * the label padding mask (fock_targets_batched.py:1012-1080);
//   * the ORCA / pyscf <-> e3nn m-ordering of a Hamiltonian, a signed
//     permutation S H S^T (fock_utils/utils_orca_out.py:402-465);
//   * a block list (SparseBlockMatrix) to CSR arrays
//     (matrix2labels_kernels.py:16-42).
// All of them are HBM-bound gathers or scatters; every output element is
// written by exactly one thread (no atomics, bit-exact).
#include "common.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace fa {

// labels[r][cols[k]] += sign * means[Z[r]][k], one thread per (row, k).
__global__ void scalar_shift_kernel(float* __restrict__ labels, int64_t ld, int64_t num_rows,
                                    const int32_t* __restrict__ Z, const float* __restrict__ means,
                                    const int32_t* __restrict__ cols, int ncols, float sign) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= num_rows * ncols) return;
  const int64_t r = i / ncols;
  const int k = static_cast<int>(i - r * ncols);
  const float m = means[static_cast<int64_t>(Z[r]) * ncols + k];
  float* p = labels + r * ld + cols[k];
  *p = *p + sign * m;
}

// mask[r][c] = cover[pair_kind[Z[rows[r]] * 100 + Z[cols[r]]]][c] (0 for pairs
// without a template), one thread per 4 bytes of a row.
__global__ void label_mask_kernel(const int32_t* __restrict__ rows, const int32_t* __restrict__ cols,
                                  const int32_t* __restrict__ Z, const int32_t* __restrict__ pair_kind,
                                  const uint8_t* __restrict__ cover, int t, int64_t num_rows,
                                  uint8_t* __restrict__ mask) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= num_rows * t) return;
  const int64_t r = i / t;
  const int c = static_cast<int>(i - r * t);
  const int kind = pair_kind[Z[rows[r]] * 100 + Z[cols[r]]];
  mask[i] = kind < 0 ? 0 : cover[static_cast<int64_t>(kind) * t + c];
}

// out[i][j] = sign[i] sign[j] H[src[i]][src[j]]: a thread per 4 consecutive
// output columns of one row.
__global__ void signed_permute_kernel(const float* __restrict__ H, int64_t n, int64_t ld_in,
                                      const int32_t* __restrict__ src, const float* __restrict__ sign,
                                      float* __restrict__ out, int64_t ld_out) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_row = (n + 3) / 4;
  if (q >= n * per_row) return;
  const int64_t i = q / per_row;
  const int64_t j0 = (q - i * per_row) * 4;
  const float si = sign[i];
  const float* hr = H + static_cast<int64_t>(src[i]) * ld_in;
  float* o = out + i * ld_out;
  for (int64_t j = j0; j < j0 + 4 && j < n; ++j) o[j] = si * sign[j] * hr[src[j]];
}

// Block b (row atom i = brow[b], column atom j = bcol[b], n_i x n_j
// row-major at data[bdo[b]]) into CSR: element (a, c) lands at
// indptr[off[i] + a] + coloff[b] + c with column off[j] + c, where coloff[b]
// is the number of columns of the blocks left of b in its block row.
__global__ void blocks_to_csr_kernel(const float* __restrict__ data, const int64_t* __restrict__ bdo,
                                     const int32_t* __restrict__ brow, const int32_t* __restrict__ bcol,
                                     const int32_t* __restrict__ off, const int64_t* __restrict__ coloff,
                                     const int64_t* __restrict__ indptr, int64_t num_blocks,
                                     float* __restrict__ csr_data, int64_t* __restrict__ csr_indices) {
  const int64_t b = blockIdx.x;
  if (b >= num_blocks) return;
  const int i = brow[b], j = bcol[b];
  const int ni = off[i + 1] - off[i], nj = off[j + 1] - off[j];
  const float* src = data + bdo[b];
  for (int e = threadIdx.x; e < ni * nj; e += blockDim.x) {
    const int a = e / nj, c = e - a * nj;
    const int64_t pos = indptr[off[i] + a] + coloff[b] + c;
    csr_data[pos] = src[e];
    csr_indices[pos] = off[j] + c;
  }
}

int grid_of(int64_t n, int64_t per, unsigned* g) {
  const int64_t blocks = (n + per - 1) / per;
  MALOQ_REQUIRE(blocks < (int64_t(1) << 31), "grid too large");
  *g = static_cast<unsigned>(blocks);
  return MALOQ_OK;
}

}  // namespace fa
}  // namespace maloq

using namespace maloq;

extern "C" int maloq_label_scalar_shift(float* labels, int64_t ld, int64_t num_rows, const int32_t* atomic_numbers,
                                        const float* means, const int32_t* cols, int ncols, float sign,
                                        void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && ncols >= 0, "negative size");
  if (num_rows == 0 || ncols == 0) return MALOQ_OK;
  MALOQ_REQUIRE(labels && atomic_numbers && means && cols, "null pointer");
  unsigned g;
  if (fa::grid_of(num_rows * ncols, 256, &g)) return MALOQ_EINVAL;
  hipLaunchKernelGGL(fa::scalar_shift_kernel, dim3(g), dim3(256), 0, static_cast<hipStream_t>(stream), labels, ld,
                     num_rows, atomic_numbers, means, cols, ncols, sign);
  return check_launch("scalar_shift_kernel");
}

extern "C" int maloq_label_mask(const int32_t* rows, const int32_t* cols, const int32_t* atomic_numbers,
                                const int32_t* pair_kind, const uint8_t* cover, int t, int64_t num_rows,
                                uint8_t* mask, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && t > 0, "bad size");
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(rows && cols && atomic_numbers && pair_kind && cover && mask, "null pointer");
  unsigned g;
  if (fa::grid_of(num_rows * t, 256, &g)) return MALOQ_EINVAL;
  hipLaunchKernelGGL(fa::label_mask_kernel, dim3(g), dim3(256), 0, static_cast<hipStream_t>(stream), rows, cols,
                     atomic_numbers, pair_kind, cover, t, num_rows, mask);
  return check_launch("label_mask_kernel");
}

extern "C" int maloq_signed_permute(const float* H, int64_t n, int64_t ld_in, const int32_t* src, const float* sign,
                                    float* out, int64_t ld_out, void* stream) {
  MALOQ_REQUIRE(n >= 0 && ld_in >= n && ld_out >= n, "bad matrix size");
  if (n == 0) return MALOQ_OK;
  MALOQ_REQUIRE(H && src && sign && out && H != out, "null or aliased pointer");
  unsigned g;
  if (fa::grid_of(n * ((n + 3) / 4), 256, &g)) return MALOQ_EINVAL;
  hipLaunchKernelGGL(fa::signed_permute_kernel, dim3(g), dim3(256), 0, static_cast<hipStream_t>(stream), H, n, ld_in,
                     src, sign, out, ld_out);
  return check_launch("signed_permute_kernel");
}

extern "C" int maloq_blocks_to_csr(const float* data, const int64_t* block_data_offsets, const int32_t* block_rows,
                                   const int32_t* block_cols, const int32_t* fock_block_offsets,
                                   const int64_t* block_col_offsets, const int64_t* indptr, int64_t num_blocks,
                                   float* csr_data, int64_t* csr_indices, void* stream) {
  MALOQ_REQUIRE(num_blocks >= 0, "num_blocks < 0");
  if (num_blocks == 0) return MALOQ_OK;
  MALOQ_REQUIRE(data && block_data_offsets && block_rows && block_cols && fock_block_offsets && block_col_offsets &&
                indptr && csr_data && csr_indices, "null pointer");
  MALOQ_REQUIRE(num_blocks < (int64_t(1) << 31), "too many blocks");
  hipLaunchKernelGGL(fa::blocks_to_csr_kernel, dim3(static_cast<unsigned>(num_blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), data, block_data_offsets, block_rows, block_cols,
                     fock_block_offsets, block_col_offsets, indptr, num_blocks, csr_data, csr_indices);
  return check_launch("blocks_to_csr_kernel");
}
