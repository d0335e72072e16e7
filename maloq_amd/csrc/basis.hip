// Fock-matrix <-> irreps-label basis transform (gfx950).
//
// HBM-bound work: every kernel stages a tile of rows (label rows, or the
// atom-pair blocks of the Fock matrix) in LDS with coalesced loads, then each
// thread produces one output column for a chunk of rows from block-local dot
// products against the Clebsch-Gordan tables (tiny, L1/L2 resident).  The
// inverse scatter is deterministic: every Fock entry is written by exactly
// one (row, column) pair, no atomics.
//
// Reference semantics: e3TensorDecomp.get_H / get_net_out
// (fock_utils/utils_tensor_decomp.py:154-169), the Triton kernels K6/K8
// (basis_transform_triton_backend.py:853-1008) and the CuPy gather/scatter
// K12/K13 (matrix2labels_kernels.py:547-800).
#include "common.h"
#include "../../include/maloq_hip.h"

namespace maloq {

constexpr int kThreads = 256;
constexpr int kChunk = 8;  // rows per thread-unit
constexpr int kMaxElements = 100;

// ---------------------------------------------------------------- labels
__global__ __launch_bounds__(kThreads) void label_transform_kernel(
    const float* __restrict__ in, int64_t R, int t_in, const int32_t* __restrict__ in_col_map,
    float* __restrict__ out, int t_out, const int32_t* __restrict__ ocol_src,
    const int32_t* __restrict__ ocol_len, const int32_t* __restrict__ ocol_woff,
    const float* __restrict__ w, int G) {
  extern __shared__ float smem[];
  float* sIn = smem;  // [G][t_in]
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * G;
  const int nrows = static_cast<int>((R - r0) < G ? (R - r0) : G);
  const int64_t n_in = static_cast<int64_t>(nrows) * t_in;
  const float* src = in + r0 * t_in;
  for (int64_t i = threadIdx.x; i < n_in; i += blockDim.x) sIn[i] = src[i];
  __syncthreads();
  const int nchunks = (nrows + kChunk - 1) / kChunk;
  const int units = nchunks * t_out;
  for (int u = threadIdx.x; u < units; u += blockDim.x) {
    const int o = u % t_out, ch = u / t_out;
    const int s = ocol_src[o], len = ocol_len[o], wo = ocol_woff[o];
    float acc[kChunk];
#pragma unroll
    for (int g = 0; g < kChunk; ++g) acc[g] = 0.f;
    const int gbase = ch * kChunk;
    for (int k = 0; k < len; ++k) {
      const float wv = w[wo + k];
      const int c = in_col_map ? in_col_map[s + k] : s + k;
#pragma unroll
      for (int g = 0; g < kChunk; ++g) {
        const int gg = gbase + g;
        if (gg < nrows) acc[g] = fmaf(sIn[gg * t_in + c], wv, acc[g]);
      }
    }
#pragma unroll
    for (int g = 0; g < kChunk; ++g) {
      const int gg = gbase + g;
      if (gg < nrows) out[(r0 + gg) * t_out + o] = acc[g];
    }
  }
}

// Locates atom-pair block r: base offset into `fock` and its row stride.
struct BlockRef {
  int64_t base;
  int64_t ld;
  int ni, nj, kind;
};

__device__ __forceinline__ BlockRef block_ref(int64_t r, int64_t ld, const int64_t* data_offsets,
                                              const int32_t* off, const int32_t* Z,
                                              const int32_t* rows, const int32_t* cols,
                                              const int32_t* pair_kind) {
  BlockRef b;
  const int i = rows[r], j = cols[r];
  const int oi = off[i], oj = off[j];
  b.ni = off[i + 1] - oi;
  b.nj = off[j + 1] - oj;
  if (data_offsets) {
    b.base = data_offsets[r];
    b.ld = b.nj;
  } else {
    b.base = static_cast<int64_t>(oi) * ld + oj;
    b.ld = ld;
  }
  b.kind = pair_kind ? pair_kind[Z[i] * kMaxElements + Z[j]] : -1;
  return b;
}

__global__ __launch_bounds__(kThreads) void fock_to_irreps_kernel(
    const float* __restrict__ fock, int64_t ld, const int64_t* __restrict__ data_offsets,
    const int32_t* __restrict__ off, const int32_t* __restrict__ Z,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ cols, int64_t R,
    const int32_t* __restrict__ pair_kind, const int32_t* __restrict__ sub_origin, int nblocks,
    const int32_t* __restrict__ block_n2, float* __restrict__ out, int t_out,
    const int32_t* __restrict__ ocol_block, const int32_t* __restrict__ ocol_len,
    const int32_t* __restrict__ ocol_woff, const float* __restrict__ w, int maxe, int G) {
  extern __shared__ float smem[];
  float* sBlk = smem;                                          // [G][maxe]
  int* sMeta = reinterpret_cast<int*>(sBlk + static_cast<int64_t>(G) * maxe);  // [G][2]: nj, kind
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * G;
  const int nrows = static_cast<int>((R - r0) < G ? (R - r0) : G);
  // One wave-sized group of threads per row loads its block.
  for (int g = threadIdx.x / 64; g < nrows; g += blockDim.x / 64) {
    const BlockRef b = block_ref(r0 + g, ld, data_offsets, off, Z, rows, cols, pair_kind);
    const int ne = b.ni * b.nj;
    for (int q = threadIdx.x % 64; q < ne; q += 64) {
      const int a = q / b.nj, c = q - a * b.nj;
      sBlk[g * maxe + q] = fock[b.base + a * b.ld + c];
    }
    if (threadIdx.x % 64 == 0) {
      sMeta[2 * g] = b.nj;
      sMeta[2 * g + 1] = b.kind;
    }
  }
  __syncthreads();
  const int nchunks = (nrows + kChunk - 1) / kChunk;
  const int units = nchunks * t_out;
  for (int u = threadIdx.x; u < units; u += blockDim.x) {
    const int o = u % t_out, ch = u / t_out;
    const int blk = ocol_block[o], len = ocol_len[o], wo = ocol_woff[o], n2 = block_n2[blk];
    for (int g = ch * kChunk; g < min(nrows, (ch + 1) * kChunk); ++g) {
      const int nj = sMeta[2 * g], kind = sMeta[2 * g + 1];
      float acc = 0.f;
      if (kind >= 0) {
        const int rr = sub_origin[(kind * nblocks + blk) * 2], cc = sub_origin[(kind * nblocks + blk) * 2 + 1];
        if (rr >= 0) {
          const float* blkp = sBlk + g * maxe + rr * nj + cc;
          int a = 0, bcol = 0;
          for (int k = 0; k < len; ++k) {
            acc = fmaf(blkp[a * nj + bcol], w[wo + k], acc);
            if (++bcol == n2) { bcol = 0; ++a; }
          }
        }
      }
      out[(r0 + g) * t_out + o] = acc;
    }
  }
}

__global__ __launch_bounds__(kThreads) void irreps_to_fock_kernel(
    const float* __restrict__ irreps, int64_t R, int t_in, float* __restrict__ fock, int64_t ld,
    const int64_t* __restrict__ data_offsets, const int32_t* __restrict__ off,
    const int32_t* __restrict__ Z, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ cols, const int32_t* __restrict__ pair_kind,
    const int32_t* __restrict__ sub_origin, int nblocks, const int32_t* __restrict__ block_n2,
    int t_h, const int32_t* __restrict__ hcol_block, const int32_t* __restrict__ hcol_pos,
    const int32_t* __restrict__ hcol_src, const int32_t* __restrict__ hcol_len,
    const int32_t* __restrict__ hcol_woff, const float* __restrict__ w, int G) {
  extern __shared__ float smem[];
  float* sIn = smem;  // [G][t_in]
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * G;
  const int nrows = static_cast<int>((R - r0) < G ? (R - r0) : G);
  const int64_t n_in = static_cast<int64_t>(nrows) * t_in;
  const float* src = irreps + r0 * t_in;
  for (int64_t i = threadIdx.x; i < n_in; i += blockDim.x) sIn[i] = src[i];
  __syncthreads();
  const int nchunks = (nrows + kChunk - 1) / kChunk;
  const int units = nchunks * t_h;
  for (int u = threadIdx.x; u < units; u += blockDim.x) {
    const int h = u % t_h, ch = u / t_h;
    const int blk = hcol_block[h], pos = hcol_pos[h], s = hcol_src[h], len = hcol_len[h],
              wo = hcol_woff[h], n2 = block_n2[blk];
    const int pa = pos / n2, pb = pos - pa * n2;
    for (int g = ch * kChunk; g < min(nrows, (ch + 1) * kChunk); ++g) {
      const BlockRef b = block_ref(r0 + g, ld, data_offsets, off, Z, rows, cols, pair_kind);
      if (b.kind < 0) continue;
      const int rr = sub_origin[(b.kind * nblocks + blk) * 2];
      const int cc = sub_origin[(b.kind * nblocks + blk) * 2 + 1];
      if (rr < 0) continue;
      float acc = 0.f;
      for (int k = 0; k < len; ++k) acc = fmaf(sIn[g * t_in + s + k], w[wo + k], acc);
      fock[b.base + static_cast<int64_t>(rr + pa) * b.ld + cc + pb] = acc;
    }
  }
}

// ------------------------------------------------------- plain copy (K12/K13)
__global__ __launch_bounds__(kThreads) void matrix2label_kernel(
    float* __restrict__ fock, int64_t ld, const int64_t* __restrict__ data_offsets,
    const int32_t* __restrict__ off, const int32_t* __restrict__ Z,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ cols, int64_t R,
    const int32_t* __restrict__ tmpl_ptr, const int32_t* __restrict__ tmpl,
    float* __restrict__ target, int64_t target_ld, int forward) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64;
  if (r >= R) return;
  const int lane = threadIdx.x % 64;
  const BlockRef b = block_ref(r, ld, data_offsets, off, Z, rows, cols, nullptr);
  const int key = Z[rows[r]] * kMaxElements + Z[cols[r]];
  float* trow = target + r * target_ld;
  for (int t = tmpl_ptr[key]; t < tmpl_ptr[key + 1]; ++t) {
    const int ra = tmpl[5 * t], rb = tmpl[5 * t + 1], ca = tmpl[5 * t + 2], cb = tmpl[5 * t + 3],
              o0 = tmpl[5 * t + 4];
    const int wdt = cb - ca, ne = (rb - ra) * wdt;
    for (int k = lane; k < ne; k += 64) {
      const int a = k / wdt, c = k - a * wdt;
      const int64_t fp = b.base + static_cast<int64_t>(ra + a) * b.ld + ca + c;
      if (forward)
        trow[o0 + k] = fock[fp];
      else
        fock[fp] = trow[o0 + k];
    }
  }
}

}  // namespace maloq

using namespace maloq;

static int rows_per_block(int row_floats, int64_t R) {
  // Keep the staged tile under 64 KB of LDS and at most 64 rows.
  int g = 64;
  while (g > kChunk && static_cast<int64_t>(g) * row_floats * 4 > 64 * 1024) g /= 2;
  (void)R;
  return g;
}

extern "C" int maloq_label_transform(const float* in, int64_t num_rows, int t_in,
                                     const int32_t* in_col_map, float* out, int t_out,
                                     const int32_t* ocol_src, const int32_t* ocol_len,
                                     const int32_t* ocol_woff, const float* w, int max_len,
                                     void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && t_in > 0 && t_out > 0, "bad sizes");
  (void)max_len;
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(in && out && ocol_src && ocol_len && ocol_woff && w, "null pointer");
  const int G = rows_per_block(t_in, num_rows);
  MALOQ_REQUIRE(static_cast<int64_t>(kChunk) * t_in * 4 <= 64 * 1024, "label width %d too large", t_in);
  const int64_t blocks = (num_rows + G - 1) / G;
  const size_t shm = static_cast<size_t>(G) * t_in * sizeof(float);
  hipLaunchKernelGGL(label_transform_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                     shm, static_cast<hipStream_t>(stream), in, num_rows, t_in, in_col_map, out,
                     t_out, ocol_src, ocol_len, ocol_woff, w, G);
  return check_launch("label_transform_kernel");
}

extern "C" int maloq_fock_to_irreps(const float* fock, int64_t ld, const int64_t* data_offsets,
                                    const int32_t* fock_block_offsets,
                                    const int32_t* atomic_numbers, const int32_t* rows,
                                    const int32_t* cols, int64_t num_rows,
                                    const int32_t* pair_kind, const int32_t* sub_origin,
                                    int nblocks, const int32_t* block_n2, float* out, int t_out,
                                    const int32_t* ocol_block, const int32_t* ocol_len,
                                    const int32_t* ocol_woff, const float* w,
                                    int max_block_elems, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && t_out > 0 && nblocks > 0, "bad sizes");
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(fock && fock_block_offsets && atomic_numbers && rows && cols && pair_kind &&
                    sub_origin && block_n2 && out && ocol_block && ocol_len && ocol_woff && w,
                "null pointer");
  MALOQ_REQUIRE(max_block_elems > 0 && max_block_elems <= 8192, "max_block_elems out of range");
  int G = 64;
  while (G > kChunk && static_cast<int64_t>(G) * (max_block_elems + 2) * 4 > 64 * 1024) G /= 2;
  const size_t shm = static_cast<size_t>(G) * max_block_elems * sizeof(float) + 2 * G * sizeof(int);
  const int64_t blocks = (num_rows + G - 1) / G;
  hipLaunchKernelGGL(fock_to_irreps_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                     shm, static_cast<hipStream_t>(stream), fock, ld, data_offsets,
                     fock_block_offsets, atomic_numbers, rows, cols, num_rows, pair_kind,
                     sub_origin, nblocks, block_n2, out, t_out, ocol_block, ocol_len, ocol_woff, w,
                     max_block_elems, G);
  return check_launch("fock_to_irreps_kernel");
}

extern "C" int maloq_irreps_to_fock(const float* irreps, int64_t num_rows, int t_in, float* fock,
                                    int64_t ld, const int64_t* data_offsets,
                                    const int32_t* fock_block_offsets,
                                    const int32_t* atomic_numbers, const int32_t* rows,
                                    const int32_t* cols, const int32_t* pair_kind,
                                    const int32_t* sub_origin, int nblocks,
                                    const int32_t* block_n2, int t_h, const int32_t* hcol_block,
                                    const int32_t* hcol_pos, const int32_t* hcol_src,
                                    const int32_t* hcol_len, const int32_t* hcol_woff,
                                    const float* w, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && t_in > 0 && t_h > 0 && nblocks > 0, "bad sizes");
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(irreps && fock && fock_block_offsets && atomic_numbers && rows && cols &&
                    pair_kind && sub_origin && block_n2 && hcol_block && hcol_pos && hcol_src &&
                    hcol_len && hcol_woff && w,
                "null pointer");
  const int G = rows_per_block(t_in, num_rows);
  MALOQ_REQUIRE(static_cast<int64_t>(kChunk) * t_in * 4 <= 64 * 1024, "irreps width %d too large", t_in);
  const size_t shm = static_cast<size_t>(G) * t_in * sizeof(float);
  const int64_t blocks = (num_rows + G - 1) / G;
  hipLaunchKernelGGL(irreps_to_fock_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                     shm, static_cast<hipStream_t>(stream), irreps, num_rows, t_in, fock, ld,
                     data_offsets, fock_block_offsets, atomic_numbers, rows, cols, pair_kind,
                     sub_origin, nblocks, block_n2, t_h, hcol_block, hcol_pos, hcol_src, hcol_len,
                     hcol_woff, w, G);
  return check_launch("irreps_to_fock_kernel");
}

extern "C" int maloq_matrix2label(float* fock, int64_t ld, const int64_t* data_offsets,
                                  const int32_t* fock_block_offsets,
                                  const int32_t* atomic_numbers, const int32_t* rows,
                                  const int32_t* cols, int64_t num_rows, const int32_t* tmpl_ptr,
                                  const int32_t* tmpl, float* target, int64_t target_ld,
                                  int forward, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0, "bad sizes");
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(fock && fock_block_offsets && atomic_numbers && rows && cols && tmpl_ptr && tmpl &&
                    target,
                "null pointer");
  const int rows_per_wg = kThreads / 64;
  const int64_t blocks = (num_rows + rows_per_wg - 1) / rows_per_wg;
  hipLaunchKernelGGL(matrix2label_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), fock, ld, data_offsets, fock_block_offsets,
                     atomic_numbers, rows, cols, num_rows, tmpl_ptr, tmpl, target, target_ld,
                     forward);
  return check_launch("matrix2label_kernel");
}
