// Fock-matrix <-> irreps-label basis transform (gfx950).
//
// The transform is block diagonal: every Clebsch-Gordan block b (one shell
// pair l1 x l2 of the label row) maps its n = (2l1+1)(2l2+1) label columns to
// the same number of irreps columns by a dense n x n matrix.  Unsorted, the
// label and irreps sides of a block occupy the same columns, so a block can be
// contracted in place.
//
// Column groups.  The host splits the unsorted label row into G groups of
// consecutive CG blocks, each narrow enough for an LDS tile (one group when the
// whole row fits).  The grid is (row tiles) x (groups): a workgroup owns TR = 32
// or 64 rows (atom pairs) of one group, TR / 8 waves, and works in three phases
// over a [TR, width] fp32 tile in LDS (odd row pitch: lane-per-row reads are
// bank-conflict free):
//   1. load: the group's columns of label/irreps rows with coalesced row
//      copies, or the group's elements of the atom-pair blocks of the Fock
//      matrix (a packed per-(group, element pair) list of (element, column),
//      in memory order, so the walk is coalesced);
//   2. contract: the group's CG blocks are split into 4 lists on the host
//      (longest-processing-time balanced); with 4 waves each wave runs one
//      list, with 8 every other block of one list.  Lane = row, so the n x n
//      block matrix is the same for all 64 lanes.  A block whose matrix is one
//      of the compiled CG programs (cg_blocks.h: its exact zeros skipped, its
//      weights literals, about a fifth of the dense FMAs and no weight loads)
//      runs that program; any other block runs the dense n x n loop with its
//      weights read into SGPRs.  A block that no row of the tile has (an
//      element pair without that shell pair) is skipped;
//   3. store: coalesced rows (through the sort permutation when the row is one
//      group) or the group's elements of the atom-pair blocks again (every Fock
//      entry belongs to one group and is written by exactly one (row, column):
//      deterministic, no atomics).
// Single-group label / irreps rows whose width is a multiple of 4 are loaded
// and stored 16 bytes (4 consecutive columns) per lane.
//
// Fock-side calls run on a row plan: maloq_basis_row_meta describes every row
// (block base, original row index, element-pair kind, block shape) once per
// structure, in row order.  The *_pairs entry points take the pair list
// instead: each workgroup describes its own rows the same way (one launch, no
// plan; the same bits).
//
// Reference semantics: e3TensorDecomp.get_H / get_net_out
// (fock_utils/utils_tensor_decomp.py:154-169), the Triton kernels K6/K8
// (basis_transform_triton_backend.py:853-1008, whose grid also runs over CG
// blocks: :1255-1438) and the CuPy gather/scatter K12/K13
// (matrix2labels_kernels.py:547-800).
#include "common.h"
#include "cg_blocks.h"
#include "../../include/maloq_hip.h"

namespace maloq {

constexpr int kThreads = 256;
constexpr int kMaxElements = 100;

namespace bt {

// Tile rows TR: 64 (8 waves, every lane a row in phase 2) where the LDS tile
// still lets as many waves share a CU as 32-row tiles would; otherwise 32 (4
// waves, the upper half-wave repeats the lower one in phase 2).  Each wave
// loads and stores 8 rows.
constexpr int kRowsPerWave = 8;
constexpr int kNarrowRows = 32, kWideRows = 64;
constexpr int kSchedLists = 4;       // CG block lists of the host schedule
__host__ __device__ constexpr int waves_of(int tr) { return tr / kRowsPerWave; }
// rows per wave per load pass (x 4 chunks of 64): half a wave's 8 rows, 16
// loads in flight per lane.  All 8 in one pass held 98 VGPRs (4 workgroups per
// CU instead of 6) and ran 20-25 % slower.
constexpr int kPassRows = kRowsPerWave / 2;
constexpr int kMaxTileBytes = 160 * 1024;
constexpr int kStaticLds = 256;      // LDS the compiler adds beyond Smem (barrier reductions)
constexpr int kMaxSkipBlocks = 64;   // CG blocks of one column group (its presence mask)

enum Side { ROWS = 0, FOCK = 1 };

// Layout of the host's tables (maloq_amd/basis_transform.py builds them):
//   sched: [0] = G; [1 + 4g ..] = (first column, width, first block, offset o_g
//     of the group's block lists) of group g; at o_g the 5 offsets (relative to
//     o_g + 5) of the group's 4 block lists, then their (global) block ids;
//   slots: [0] = kinds K, [1] = G, [2 + g] = the largest rectangle (nr * nc) of
//     group g; [2 + G + g*K + k] = the rectangle of (group g, kind k) in its
//     atom-pair block, r0 | nr << 8 | c0 << 16 | nc << 24 (rows r0 .. r0+nr-1,
//     columns c0 .. c0+nc-1; nr = 0: none); [2 + G + G*K + g*K + k] = offset of
//     its column table: nr*nc entries, row-major, the tile column of each
//     element or -1.  With one group the rectangle is the whole block and the
//     tables are rows of maxe entries from 3 + 2K on (kind k's at 3 + 2K + k*maxe);
//   kind_blocks: [G*K, 2] presence masks, bit i = the group's i-th CG block.
constexpr int kGroupWords = 4;
constexpr int kSlotHead = 2;

struct Args {
  const float* in;          // ROWS input [R, t]
  const int32_t* perm_in;   // input column j -> unsorted column, or null (one group only)
  float* out;               // ROWS output [R, t]
  const int32_t* perm_out;  // output column j <- unsorted column, or null (one group only)
  int64_t R;
  int t, tp;                // row width, LDS row pitch (odd, >= the widest group)
  int ngroups, gcols;       // column groups, widest group
  // Fock side
  float* fock;
  int64_t ld;               // dense row stride, or 0 for block-list storage
  const int4* meta;         // [R] row plan (maloq_basis_row_meta), processing order, or
                            // null: the kernel describes its rows itself from the pair list
  const int64_t* data_offsets;  // pair list (meta null): block-list bases, or null (dense)
  const int32_t* off;           //   [atoms + 1] first orbital of each atom
  const int32_t* Z;             //   [atoms] atomic numbers
  const int32_t* rows;          //   [R] atom i of pair r
  const int32_t* cols;          //   [R] atom j of pair r
  const int32_t* pair_kind;     //   [100 * 100] element-pair kind, or -1
  const int32_t* slots;     // per (group, kind) element rectangles (layout above)
  int maxe;                 // largest n_i * n_j of the template
  const uint32_t* kind_blocks;  // [G * kinds, 2]: CG blocks present (bit: group-local block), or null
  // CG tables
  int nblocks;
  const int32_t* blocks;    // [nblocks, 4]: n, first column, weight offset, CG program or -1
  const float* w;
  const int32_t* sched;     // column groups and block lists (layout above)
};

// One column group, read from sched (uniform).
struct Group {
  int c0, width, b0, lists;
};

// Per tile row, for the workgroup's column group: the row's rectangle of its
// atom-pair block (element k of the rectangle, i = k / nc, j = k % nc, is at
// base + i * rs + j) and the rectangle's column table.
template <int TR>
struct Smem {
  int64_t base[TR];  // block base + r0 * rs + c0
  int row[TR];       // original row index
  int kind[TR];
  int cnt[TR];       // nr * nc (0: nothing of this group)
  int nc[TR];        // 0 where the rectangle's rows are contiguous (nc = rs): offset k
  float rnc[TR];     // 1 / nc, 0 where nc is
  int rs[TR];        // row stride: ld (dense) or n_j (block list)
  int lo[TR];        // first entry of the column table
};

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// The CG tables are read through the constant address space: uniform
// addresses there become scalar loads (no vector load plus readfirstlane).
template <class T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* konst(const T* p) {
  return (const __attribute__((address_space(4))) T*)(p);
}

// Row plan entry of pair r: int4 (base lo, base hi, r, (kind + 1) | n_i << 16 |
// n_j << 24).
__device__ __forceinline__ int4 describe_row(int64_t r, int64_t ld, const int64_t* __restrict__ data_offsets,
                                             const int32_t* __restrict__ off, const int32_t* __restrict__ Z,
                                             const int32_t* __restrict__ rows, const int32_t* __restrict__ cols,
                                             const int32_t* __restrict__ pair_kind, int maxe) {
  const int i = rows[r], j = cols[r];
  const int oi = off[i], oj = off[j];
  const int ni = off[i + 1] - oi, nj = off[j + 1] - oj;
  const int64_t base = data_offsets ? data_offsets[r] : static_cast<int64_t>(oi) * ld + oj;
  int kind = pair_kind[Z[i] * kMaxElements + Z[j]];
  // a block larger than the template's rows cannot be one of its element pairs
  if (ni > 255 || nj > 255 || ni * nj > maxe) kind = -1;
  return make_int4(static_cast<int>(base & 0xffffffff), static_cast<int>(base >> 32), static_cast<int>(r),
                   (kind + 1) | ((ni & 255) << 16) | ((nj & 255) << 24));
}

__global__ __launch_bounds__(kThreads) void row_meta_kernel(
    int64_t R, int64_t ld, const int64_t* __restrict__ data_offsets,
    const int32_t* __restrict__ off, const int32_t* __restrict__ Z,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ cols,
    const int32_t* __restrict__ pair_kind, int maxe, int4* __restrict__ meta) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (r >= R) return;
  meta[r] = describe_row(r, ld, data_offsets, off, Z, rows, cols, pair_kind, maxe);
}

// Element-pair kinds of the slot table, or 0 if it was built for another
// number of groups (both header words read unconditionally: one scalar load).
__device__ __forceinline__ int slot_kinds(const Args& a) {
  const auto* sl = konst(a.slots);
  const int k = sl[0], groups = sl[1];
  return groups == a.ngroups ? k : 0;
}

template <int TR, bool PAIRS>
__device__ __forceinline__ void load_meta(const Args& a, Smem<TR>& s, int64_t r0, int nrows, int grp) {
  const int g = threadIdx.x;
  if (g >= TR) return;
  if (g >= nrows) {
    s.base[g] = 0;
    s.kind[g] = -1;
    s.cnt[g] = 0;
    s.row[g] = -1;
    s.nc[g] = 0;
    s.rnc[g] = 0.f;
    s.rs[g] = 0;
    s.lo[g] = 0;
    return;
  }
  // from the plan, or (PAIRS) described here from the pair list: the plan's
  // entry r is the description of pair r
  int4 m;
  if constexpr (PAIRS)
    m = describe_row(r0 + g, a.ld, a.data_offsets, a.off, a.Z, a.rows, a.cols, a.pair_kind, a.maxe);
  else
    m = a.meta[r0 + g];
  // the slot table's header after the row loads are issued (its scalar load
  // overlaps them)
  const int kinds = slot_kinds(a);
  int64_t base = static_cast<int64_t>(static_cast<uint32_t>(m.x)) | (static_cast<int64_t>(m.y) << 32);
  s.row[g] = m.z;
  int kind = (m.w & 0xffff) - 1;
  const int ni = (m.w >> 16) & 255, nj = (m.w >> 24) & 255;
  if (kind >= kinds) kind = -1;  // a pair_kind entry past the slot table: no template
  const int rs = a.ld ? static_cast<int>(a.ld) : nj;
  int cnt = 0, nc = 0, lo = 0;
  if (kind >= 0 && a.ngroups == 1) {
    // one group: the whole block, and the kind's table is row `kind` of maxe
    // entries (no lookup before the gather; n_i * n_j <= maxe)
    cnt = ni * nj;
    nc = nj == rs ? 0 : nj;
    lo = kSlotHead + 1 + 2 * kinds + kind * a.maxe;
  } else if (kind >= 0) {
    const int32_t* p = a.slots + kSlotHead + a.ngroups + grp * kinds + kind;
    const uint32_t rect = static_cast<uint32_t>(p[0]);
    lo = p[a.ngroups * kinds];
    const int rr = rect & 255, nr = (rect >> 8) & 255, cc = (rect >> 16) & 255, w = rect >> 24;
    // a rectangle outside the row's actual block reads and writes nothing
    if (nr > 0 && w > 0 && rr + nr <= ni && cc + w <= nj) {
      cnt = nr * w;
      nc = w == rs ? 0 : w;
      base += static_cast<int64_t>(rr) * rs + cc;
    }
  }
  s.kind[g] = kind;
  s.base[g] = base;
  s.cnt[g] = cnt;
  s.nc[g] = nc;
  s.rnc[g] = nc ? 1.0f / static_cast<float>(nc) : 0.f;
  s.rs[g] = rs;
  s.lo[g] = lo;
}

// Offset of element k = i * nc + j of tile row g's rectangle from its base.
// i = floor((k + 1/2) / nc) in fp32 is exact: the quotient's distance to the
// nearest integer is >= 1/(2 nc) >= 2^-9, far above the rounding error for
// k < 2^16.  i * rs < 255 * 2^23 fits 32 bits.  Rows stored contiguously
// (nc = 0, rnc = 0) give i = 0 and the offset k.
template <int TR>
__device__ __forceinline__ int elem_offset(const Smem<TR>& s, int g, int k) {
  const int i = static_cast<int>((static_cast<float>(k) + 0.5f) * s.rnc[g]);
  return i * s.rs[g] + (k - i * s.nc[g]);
}

// Original row index of tile row g.
template <bool PLAN, int TR>
__device__ __forceinline__ int64_t row_of(const Smem<TR>& s, int64_t r0, int g) {
  if constexpr (PLAN)
    return s.row[g];
  else
    return r0 + g;
}

// Whether any row of a wave's pass has a strided rectangle (nc != 0); uniform.
template <int NW, int TR>
__device__ __forceinline__ bool strided_pass(const Smem<TR>& s, int wave, int i0) {
  int any = 0;
#pragma unroll
  for (int i = 0; i < kPassRows; ++i) any |= s.nc[wave + NW * (i0 + i)];
  return uniform(any) != 0;
}

// A tile row's rectangle, read once per pass into scalar registers (the row is
// the same for the whole wave).
struct RowRect {
  int64_t base;
  int cnt, nc, rs, lo;
  float rnc;
};

template <int TR>
__device__ __forceinline__ RowRect row_rect(const Smem<TR>& s, int g) {
  RowRect r;
  r.base = uniform64(s.base[g]);
  r.cnt = uniform(s.cnt[g]);
  r.nc = uniform(s.nc[g]);
  r.rs = uniform(s.rs[g]);
  r.lo = uniform(s.lo[g]);
  r.rnc = __int_as_float(uniform(__float_as_int(s.rnc[g])));
  return r;
}

// Offset of element k of a rectangle from its base (see elem_offset).
template <bool STRIDED>
__device__ __forceinline__ int rect_offset(const RowRect& r, int k) {
  if constexpr (!STRIDED) return k;
  const int i = static_cast<int>((static_cast<float>(k) + 0.5f) * r.rnc);
  return i * r.rs + (k - i * r.nc);
}

// One gather pass: kPassRows rows x 256 rectangle elements, all loads in
// flight, then dropped into their tile columns.  Every load is issued
// unconditionally (lanes past a rectangle's end read its first table entry
// and fock[0], both in bounds), so no branch stands between them.  !STRIDED: every row's rectangle is contiguous (element k at base + k).
template <int NW, bool STRIDED, int TR>
__device__ __forceinline__ void gather_pass(const Args& a, const Smem<TR>& s, float* tile, int wave, int lane,
                                            int k0, int i0) {
  float v[kPassRows][4];
  int col[kPassRows][4];
#pragma unroll
  for (int i = 0; i < kPassRows; ++i) {
    const int g = wave + NW * (i0 + i);
    const RowRect r = row_rect(s, g);
    const int32_t* slot = a.slots + r.lo;
    const float* blk = a.fock + r.base;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
      const int k = k0 + ch * 64 + lane;
      const bool ok = k < r.cnt;
      const int c = slot[ok ? k : 0];
      // lanes past the rectangle read fock[0] (a block base may lie past the
      // matrix when its atom has no orbitals)
      v[i][ch] = *(ok ? blk + rect_offset<STRIDED>(r, k) : a.fock);
      col[i][ch] = ok ? c : -1;
    }
  }
#pragma unroll
  for (int i = 0; i < kPassRows; ++i) {
    const int g = wave + NW * (i0 + i);
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
      if (col[i][ch] >= 0) tile[g * a.tp + col[i][ch]] = v[i][ch];
  }
}

// One scatter pass (the inverse of gather_pass).
template <int NW, bool STRIDED, int TR>
__device__ __forceinline__ void scatter_pass(const Args& a, const Smem<TR>& s, const float* tile, int wave,
                                             int lane, int k0, int i0) {
  int col[kPassRows][4];
#pragma unroll
  for (int i = 0; i < kPassRows; ++i) {
    const RowRect r = row_rect(s, wave + NW * (i0 + i));
    const int32_t* slot = a.slots + r.lo;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
      const int k = k0 + ch * 64 + lane;
      const bool ok = k < r.cnt;
      const int c = slot[ok ? k : 0];
      col[i][ch] = ok ? c : -1;
    }
  }
#pragma unroll
  for (int i = 0; i < kPassRows; ++i) {
    const int g = wave + NW * (i0 + i);
    const RowRect r = row_rect(s, g);
    float* blk = a.fock + r.base;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
      const int k = k0 + ch * 64 + lane;
      if (col[i][ch] >= 0) blk[rect_offset<STRIDED>(r, k)] = tile[g * a.tp + col[i][ch]];
    }
  }
}

template <int SIDE, bool PLAN, int TR>
__device__ __forceinline__ void load_tile(const Args& a, const Smem<TR>& s, float* tile, int64_t r0,
                                          int nrows, const Group& gr, int gmax) {
  constexpr int NW = waves_of(TR);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if constexpr (SIDE == ROWS) {
    if ((a.t & 3) == 0 && a.ngroups == 1) {
      // one group of 16-byte aligned width: each lane loads 4 consecutive columns
      for (int c4 = 4 * lane; c4 < a.t; c4 += 256) {
        int dc[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) dc[k] = a.perm_in ? a.perm_in[c4 + k] : c4 + k;
        for (int i0 = 0; i0 < kRowsPerWave; i0 += kPassRows) {
          float4 v[kPassRows];
#pragma unroll
          for (int i = 0; i < kPassRows; ++i) {
            const int g = wave + NW * (i0 + i);
            v[i] = *reinterpret_cast<const float4*>(a.in + (g < nrows ? row_of<PLAN>(s, r0, g) : r0) * a.t + c4);
          }
#pragma unroll
          for (int i = 0; i < kPassRows; ++i) {
            const int g = wave + NW * (i0 + i);
            if (g < nrows) {
              float* tr = tile + g * a.tp;
              tr[dc[0]] = v[i].x;
              tr[dc[1]] = v[i].y;
              tr[dc[2]] = v[i].z;
              tr[dc[3]] = v[i].w;
            }
          }
        }
      }
      return;
    }
    // wave w copies rows w, w + NW, ... in passes of kPassRows rows x 256
    // columns of the group (coalesced along the row), all loads of a pass in
    // flight.  The permutation applies only to a row of one group (c0 = 0).
    for (int cb = 0; cb < gr.width; cb += 256) {
      int dc[4];
#pragma unroll
      for (int ch = 0; ch < 4; ++ch) {
        const int c = cb + ch * 64 + lane;
        dc[ch] = c < gr.width ? (a.perm_in ? a.perm_in[c] : c) : -1;
      }
      for (int i0 = 0; i0 < kRowsPerWave; i0 += kPassRows) {
        float v[kPassRows][4];
#pragma unroll
        for (int i = 0; i < kPassRows; ++i)
#pragma unroll
          for (int ch = 0; ch < 4; ++ch) {
            const int g = wave + NW * (i0 + i), c = cb + ch * 64 + lane;
            const bool ok = g < nrows && c < gr.width;
            const float x = a.in[ok ? row_of<PLAN>(s, r0, g) * a.t + gr.c0 + c : 0];
            v[i][ch] = ok ? x : 0.f;
          }
#pragma unroll
        for (int i = 0; i < kPassRows; ++i)
#pragma unroll
          for (int ch = 0; ch < 4; ++ch) {
            const int g = wave + NW * (i0 + i);
            if (g < nrows && dc[ch] >= 0) tile[g * a.tp + dc[ch]] = v[i][ch];
          }
      }
    }
  } else {
    // Zero the tile (label columns the element pair lacks stay zero), then
    // wave w walks the group's rectangles of the atom-pair blocks of rows w,
    // w + NW, ... (row-major: memory order, coalesced), passes of kPassRows
    // rows x 256 elements, and drops every element into its tile column.  The
    // address of element k depends on k alone, so the Fock and table loads of
    // a pass are in flight together.
    {
      const int n = TR * a.tp, n4 = n >> 2;
      float4* t4 = reinterpret_cast<float4*>(tile);
      for (int i = threadIdx.x; i < n4; i += NW * 64) t4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (threadIdx.x < (n & 3)) tile[4 * n4 + threadIdx.x] = 0.f;
    }
    __syncthreads();
    for (int k0 = 0; k0 < gmax; k0 += 256) {
      for (int i0 = 0; i0 < kRowsPerWave; i0 += kPassRows) {
        // a pass whose rectangles are all stored as contiguous rows (one
        // group over block-list storage) uses the offset k itself
        if (strided_pass<NW>(s, wave, i0))
          gather_pass<NW, true>(a, s, tile, wave, lane, k0, i0);
        else
          gather_pass<NW, false>(a, s, tile, wave, lane, k0, i0);
      }
    }
  }
}

template <int SIDE, bool PLAN, int TR>
__device__ __forceinline__ void store_tile(const Args& a, const Smem<TR>& s, const float* tile,
                                           int64_t r0, int nrows, const Group& gr, int gmax) {
  constexpr int NW = waves_of(TR);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if constexpr (SIDE == ROWS) {
    if ((a.t & 3) == 0 && a.ngroups == 1) {
      // one group of 16-byte aligned width: each lane stores 4 consecutive columns
      for (int c4 = 4 * lane; c4 < a.t; c4 += 256) {
        int sc[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) sc[k] = a.perm_out ? a.perm_out[c4 + k] : c4 + k;
        for (int g = wave; g < nrows; g += NW) {
          const float* tr = tile + g * a.tp;
          *reinterpret_cast<float4*>(a.out + row_of<PLAN>(s, r0, g) * a.t + c4) =
              make_float4(tr[sc[0]], tr[sc[1]], tr[sc[2]], tr[sc[3]]);
        }
      }
      return;
    }
    for (int c = lane; c < gr.width; c += 64) {
      const int sc = a.perm_out ? a.perm_out[c] : c;
      for (int g = wave; g < nrows; g += NW)
        a.out[row_of<PLAN>(s, r0, g) * a.t + gr.c0 + c] = tile[g * a.tp + sc];
    }
  } else {
    // every element of the group's rectangle of every atom-pair block, in
    // memory order.  A row's rectangle base and table start are the same for
    // the whole wave (scalar registers); the per-element addresses are offsets
    // from them.  Past a rectangle's end the table read is of its first entry
    // (rows past the tile's end have an empty rectangle at 0, inside the
    // table) and nothing is stored.
    for (int k0 = 0; k0 < gmax; k0 += 256) {
      for (int i0 = 0; i0 < kRowsPerWave; i0 += kPassRows) {
        if (strided_pass<NW>(s, wave, i0))
          scatter_pass<NW, true>(a, s, tile, wave, lane, k0, i0);
        else
          scatter_pass<NW, false>(a, s, tile, wave, lane, k0, i0);
      }
    }
  }
}

// The group's columns of the tile's rows, all zero, straight to the output.
template <int TR>
__device__ __forceinline__ void store_zero_rows(const Args& a, const Smem<TR>& s, int64_t r0, int nrows,
                                                const Group& gr) {
  constexpr int NW = waves_of(TR);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int g = wave; g < nrows; g += NW) {
    float* orow = a.out + row_of<true>(s, r0, g) * a.t + gr.c0;  // (zeros need no permutation)
    for (int c = lane; c < gr.width; c += 64) orow[c] = 0.f;
  }
}

// y = W x for one CG block of one row, in place; W row-major [N][N].
template <int N>
__device__ __forceinline__ void contract(float* row, const float* __restrict__ W) {
  float x[N];
#pragma unroll
  for (int k = 0; k < N; ++k) x[k] = row[k];
  if constexpr (N <= 25) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      float y = 0.f;
#pragma unroll
      for (int k = 0; k < N; ++k) y = fmaf(W[j * N + k], x[k], y);
      row[j] = y;
    }
  } else {
    for (int j = 0; j < N; ++j) {
      float y = 0.f;
#pragma unroll
      for (int k = 0; k < N; ++k) y = fmaf(W[j * N + k], x[k], y);
      row[j] = y;
    }
  }
}

// DENSE: the tables may hold blocks without a compiled program (read from
// a.w); otherwise every block has one and the dense loops (and their
// registers) are compiled out.
template <bool SKIP, bool DENSE, int TR>
__device__ __forceinline__ void contract_tile(const Args& a, const Smem<TR>& s, float* tile, const Group& gr,
                                              int grp, int kinds) {
  // wave w runs list w % 4 of the group's schedule: all of it with 4 waves,
  // the entries w / 4, w / 4 + 2, ... with 8 (each list is in descending cost
  // order, so the two halves cost about the same)
  constexpr int STEP = waves_of(TR) / kSchedLists;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const auto* sched = konst(a.sched + gr.lists);
  const auto* blk = konst(a.blocks);
  const int list = wave % kSchedLists;
  const int beg = uniform(sched[list] + wave / kSchedLists), end = uniform(sched[list + 1]);
  const auto* ids = sched + kSchedLists + 1;
  // lane = row; with 32 rows the upper half-wave repeats the lower one (same
  // reads, same values written)
  float* row = tile + (lane % TR) * a.tp;
  uint32_t have0 = 0xffffffffu, have1 = 0xffffffffu;  // the group's CG blocks this lane's row has
  if constexpr (SKIP) {
    const int kind = s.kind[lane % TR];
    const uint32_t* m = a.kind_blocks + 2 * (static_cast<int64_t>(grp) * kinds + (kind >= 0 ? kind : 0));
    have0 = kind >= 0 ? m[0] : 0u;
    have1 = kind >= 0 ? m[1] : 0u;
  }
  // block ids two ahead, block entries one ahead: the scalar loads of the next
  // blocks are in flight while the current block's program runs
  int b0 = beg < end ? ids[beg] : 0;
  int b1 = beg + STEP < end ? ids[beg + STEP] : 0;
  int en = 0, ec = 0, ew = 0, ep = -1;
  if (beg < end) { en = blk[4 * b0]; ec = blk[4 * b0 + 1]; ew = blk[4 * b0 + 2]; ep = blk[4 * b0 + 3]; }
  for (int p = beg; p < end; p += STEP) {
    const int b = uniform(b0);
    const int n = uniform(en), c0 = uniform(ec), woff = uniform(ew), prog = uniform(ep);
    if (p + STEP < end) { en = blk[4 * b1]; ec = blk[4 * b1 + 1]; ew = blk[4 * b1 + 2]; ep = blk[4 * b1 + 3]; }
    b0 = b1;
    if (p + 2 * STEP < end) b1 = ids[p + 2 * STEP];
    if constexpr (SKIP) {
      const int bl = b - gr.b0;  // group-local block, < kMaxSkipBlocks
      const bool mine = ((bl < 32 ? have0 >> bl : have1 >> (bl - 32)) & 1u) != 0;
      if (__builtin_amdgcn_ballot_w64(mine) == 0) continue;  // no row of the tile has block b
    }
    float* rb = row + (c0 - gr.c0);
    if (prog >= 0) {
      cg::run(prog, rb);
      continue;
    }
    if constexpr (!DENSE) continue;  // excluded by the host (w == NULL only with every program set)
    const float* W = a.w + woff;
    switch (n) {
      case 1: contract<1>(rb, W); break;
      case 3: contract<3>(rb, W); break;
      case 5: contract<5>(rb, W); break;
      case 7: contract<7>(rb, W); break;
      case 9: contract<9>(rb, W); break;
      case 15: contract<15>(rb, W); break;
      case 21: contract<21>(rb, W); break;
      case 25: contract<25>(rb, W); break;
      case 35: contract<35>(rb, W); break;
      case 49: contract<49>(rb, W); break;
      default: break;  // rejected on the host
    }
  }
}

// Waves per SIMD each variant is compiled for.  Programs only: registers
// capped as far as they go without spills (the 25 KB tile of a 196-column row
// allows six 4-wave workgroups per CU, its 50 KB 64-row tile three 8-wave
// ones).  With the dense loops the compiler's own choice is faster (the
// 49 x 49 loop needs its registers).
template <int IN, int OUT, bool DENSE>
struct MinWaves {
  static constexpr int value = DENSE ? 1 : (IN == ROWS ? (OUT == ROWS ? 6 : 5) : 4);
};

// IN/OUT: the two sides; PLAN: rows come from the row plan (Fock-side calls);
// DENSE: see contract_tile; TR: tile rows; PAIRS: Fock side without a plan
// (its own instantiation: describing rows costs the plan path no registers).
// blockIdx.x: row tile, blockIdx.y: column group.
template <int IN, int OUT, bool DENSE, int TR, bool PAIRS = false>
__global__ __launch_bounds__(waves_of(TR) * 64, (MinWaves<IN, OUT, DENSE>::value)) void transform_kernel(Args a) {
  constexpr bool PLAN = IN == FOCK || OUT == FOCK;
  extern __shared__ __attribute__((aligned(16))) float tile[];  // [TR][tp]
  __shared__ Smem<TR> s;
  const int grp = blockIdx.y;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * TR;
  const int nrows = static_cast<int>((a.R - r0) < TR ? (a.R - r0) : TR);
  // The row descriptions are loading before any table header is read; the
  // headers are read unconditionally (the host's tables have ngroups groups)
  // and checked after, so their scalar loads overlap the row loads.
  if constexpr (PLAN) load_meta<TR, PAIRS>(a, s, r0, nrows, grp);
  const auto* sd = konst(a.sched);
  const int sched_groups = sd[0];
  Group gr;
  gr.c0 = sd[1 + kGroupWords * grp];
  gr.width = sd[2 + kGroupWords * grp];
  gr.b0 = sd[3 + kGroupWords * grp];
  gr.lists = sd[4 + kGroupWords * grp];
  int kinds = 0, gmax = 0;
  if constexpr (PLAN) {
    kinds = slot_kinds(a);
    gmax = konst(a.slots)[kSlotHead + grp];
  }
  // tables that disagree with the launch (another decomposition's) do nothing
  if (sched_groups != a.ngroups || gr.width > a.gcols || gr.c0 + gr.width > a.t) return;
  if constexpr (PLAN) {
    // a tile none of whose rows has an element in this group: its label
    // columns are zero (Fock -> irreps stores them directly), and irreps ->
    // Fock writes nothing
    if (__syncthreads_or(threadIdx.x < TR && s.cnt[threadIdx.x] > 0) == 0) {
      if constexpr (OUT == ROWS) store_zero_rows<TR>(a, s, r0, nrows, gr);
      return;
    }
  }
  load_tile<IN, PLAN>(a, s, tile, r0, nrows, gr, gmax);
  __syncthreads();
  if (PLAN && a.kind_blocks != nullptr)
    contract_tile<true, DENSE>(a, s, tile, gr, grp, kinds);
  else
    contract_tile<false, DENSE>(a, s, tile, gr, grp, kinds);
  __syncthreads();
  store_tile<OUT, PLAN>(a, s, tile, r0, nrows, gr, gmax);
}

}  // namespace bt

// ------------------------------------------------------- plain copy (K12/K13)
__device__ __forceinline__ void block_base(int64_t r, int64_t ld, const int64_t* data_offsets,
                                           const int32_t* off, const int32_t* rows,
                                           const int32_t* cols, int64_t* base, int64_t* ldb) {
  const int i = rows[r], j = cols[r];
  const int oi = off[i], oj = off[j];
  if (data_offsets) {
    *base = data_offsets[r];
    *ldb = off[j + 1] - oj;
  } else {
    *base = static_cast<int64_t>(oi) * ld + oj;
    *ldb = ld;
  }
}

__global__ __launch_bounds__(kThreads) void matrix2label_kernel(
    float* __restrict__ fock, int64_t ld, const int64_t* __restrict__ data_offsets,
    const int32_t* __restrict__ off, const int32_t* __restrict__ Z,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ cols, int64_t R,
    const int32_t* __restrict__ tmpl_ptr, const int32_t* __restrict__ tmpl,
    float* __restrict__ target, int64_t target_ld, int forward) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64;
  if (r >= R) return;
  const int lane = threadIdx.x % 64;
  int64_t base, ldb;
  block_base(r, ld, data_offsets, off, rows, cols, &base, &ldb);
  const int key = Z[rows[r]] * kMaxElements + Z[cols[r]];
  float* trow = target + r * target_ld;
  for (int t = tmpl_ptr[key]; t < tmpl_ptr[key + 1]; ++t) {
    const int ra = tmpl[5 * t], rb = tmpl[5 * t + 1], ca = tmpl[5 * t + 2], cb = tmpl[5 * t + 3],
              o0 = tmpl[5 * t + 4];
    const int wdt = cb - ca, ne = (rb - ra) * wdt;
    for (int k = lane; k < ne; k += 64) {
      const int a = k / wdt, c = k - a * wdt;
      const int64_t fp = base + static_cast<int64_t>(ra + a) * ldb + ca + c;
      if (forward)
        trow[o0 + k] = fock[fp];
      else
        fock[fp] = trow[o0 + k];
    }
  }
}

}  // namespace maloq

using namespace maloq;

namespace {

int check_tables(int t, int nblocks, const int32_t* blocks, const float* w, const int32_t* sched, int ngroups,
                 int gcols) {
  MALOQ_REQUIRE(t > 0 && nblocks > 0, "bad sizes (t=%d, nblocks=%d)", t, nblocks);
  MALOQ_REQUIRE(blocks && sched, "null CG table");  // w may be NULL: every block has a program
  MALOQ_REQUIRE(ngroups >= 1 && ngroups <= nblocks && ngroups <= 65535,
                "column groups %d outside 1..min(nblocks=%d, 65535)", ngroups, nblocks);
  MALOQ_REQUIRE(gcols >= 1 && gcols <= t && (ngroups > 1 || gcols == t),
                "widest column group %d does not fit the row width %d (%d groups)", gcols, t, ngroups);
  // a 32-row tile of the widest group and its row descriptors in one CU's LDS
  MALOQ_REQUIRE(static_cast<int64_t>(bt::kNarrowRows) * ((gcols | 1) * 4) + sizeof(bt::Smem<bt::kNarrowRows>) +
                        bt::kStaticLds <=
                    bt::kMaxTileBytes,
                "column group of %d columns too wide for one LDS tile (split the row into narrower groups)", gcols);
  return MALOQ_OK;
}

int check_perms(int ngroups, const int32_t* perm_in, const int32_t* perm_out) {
  MALOQ_REQUIRE(ngroups == 1 || (perm_in == nullptr && perm_out == nullptr),
                "a column permutation needs rows of one column group (got %d groups): permute separately",
                ngroups);
  return MALOQ_OK;
}

bt::Args base_args(int64_t R, int t, int nblocks, const int32_t* blocks, const float* w,
                   const int32_t* sched, int ngroups, int gcols) {
  bt::Args a{};
  a.R = R;
  a.t = t;
  a.tp = gcols | 1;
  a.ngroups = ngroups;
  a.gcols = gcols;
  a.nblocks = nblocks;
  a.blocks = blocks;
  a.w = w;
  a.sched = sched;
  return a;
}

int set_fock_side(bt::Args& a, float* fock, int64_t ld, const int32_t* row_meta,
                  const int32_t* slots, int maxe, const uint32_t* kind_blocks) {
  MALOQ_REQUIRE(fock && row_meta && slots, "null pointer");
  MALOQ_REQUIRE(ld >= 0 && ld < (int64_t(1) << 23), "dense Fock row stride %lld out of range",
                static_cast<long long>(ld));
  MALOQ_REQUIRE(maxe > 0 && maxe <= 65535, "largest block size %d out of range", maxe);
  MALOQ_REQUIRE((reinterpret_cast<uintptr_t>(row_meta) & 15) == 0, "row_meta must be 16-byte aligned");
  a.fock = fock;
  a.ld = ld;
  a.meta = reinterpret_cast<const int4*>(row_meta);
  a.slots = slots;
  a.maxe = maxe;
  a.kind_blocks = kind_blocks;
  return MALOQ_OK;
}

// Fock side given as the pair list itself (no row plan): the kernel describes
// each tile's rows as maloq_basis_row_meta would.
int set_fock_pairs(bt::Args& a, float* fock, int64_t ld, const int64_t* data_offsets, const int32_t* off,
                   const int32_t* Z, const int32_t* rows, const int32_t* cols, int64_t num_rows,
                   const int32_t* pair_kind, const int32_t* slots, int maxe, const uint32_t* kind_blocks) {
  MALOQ_REQUIRE(num_rows < (int64_t(1) << 31), "bad number of rows");
  MALOQ_REQUIRE(fock && off && Z && rows && cols && pair_kind && slots, "null pointer");
  MALOQ_REQUIRE(data_offsets || (ld > 0 && ld < (int64_t(1) << 23)), "dense Fock row stride %lld out of range",
                static_cast<long long>(ld));
  MALOQ_REQUIRE(maxe > 0 && maxe <= 65535, "largest block size %d out of range", maxe);
  a.fock = fock;
  a.ld = data_offsets ? 0 : ld;
  a.meta = nullptr;
  a.data_offsets = data_offsets;
  a.off = off;
  a.Z = Z;
  a.rows = rows;
  a.cols = cols;
  a.pair_kind = pair_kind;
  a.slots = slots;
  a.maxe = maxe;
  a.kind_blocks = kind_blocks;
  return MALOQ_OK;
}

// Waves of TR-row workgroups that fit on one CU by LDS (tile + Smem), at most
// 24 (the register budget of the program-only variants).
template <int TR>
int resident_waves(int tp) {
  const int64_t lds = static_cast<int64_t>(TR) * tp * 4 + static_cast<int64_t>(sizeof(bt::Smem<TR>)) + bt::kStaticLds;
  const int nw = bt::waves_of(TR);
  int64_t wgs = bt::kMaxTileBytes / lds;
  if (wgs * nw > 24) wgs = 24 / nw;
  return static_cast<int>(wgs * nw);
}

template <int IN, int OUT, int TR, bool PAIRS>
int launch_tiles(const bt::Args& a, void* stream, const char* name) {
  const int64_t tiles = (a.R + TR - 1) / TR;
  MALOQ_REQUIRE(tiles < (int64_t(1) << 31), "too many rows");
  const size_t shm = static_cast<size_t>(TR) * a.tp * sizeof(float);
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(a.ngroups)), block(bt::waves_of(TR) * 64);
  if (a.w != nullptr)
    hipLaunchKernelGGL((bt::transform_kernel<IN, OUT, true, TR, PAIRS>), grid, block, shm,
                       static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL((bt::transform_kernel<IN, OUT, false, TR, PAIRS>), grid, block, shm,
                       static_cast<hipStream_t>(stream), a);
  return check_launch(name);
}

// 64-row tiles wherever they keep as many waves resident as 32-row tiles.
template <int IN, int OUT, bool PAIRS = false>
int launch_transform(const bt::Args& a, void* stream, const char* name) {
  if (resident_waves<bt::kWideRows>(a.tp) >= resident_waves<bt::kNarrowRows>(a.tp))
    return launch_tiles<IN, OUT, bt::kWideRows, PAIRS>(a, stream, name);
  return launch_tiles<IN, OUT, bt::kNarrowRows, PAIRS>(a, stream, name);
}

}  // namespace

extern "C" int maloq_label_transform(const float* in, const int32_t* perm_in, float* out,
                                     const int32_t* perm_out, int64_t num_rows, int t,
                                     int nblocks, const int32_t* blocks, const float* w,
                                     const int32_t* sched, int ngroups, int group_cols, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0, "bad sizes");
  if (int rc = check_tables(t, nblocks, blocks, w, sched, ngroups, group_cols)) return rc;
  if (int rc = check_perms(ngroups, perm_in, perm_out)) return rc;
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(in && out, "null pointer");
  bt::Args a = base_args(num_rows, t, nblocks, blocks, w, sched, ngroups, group_cols);
  a.in = in;
  a.perm_in = perm_in;
  a.out = out;
  a.perm_out = perm_out;
  return launch_transform<bt::ROWS, bt::ROWS>(a, stream, "label transform");
}

extern "C" int maloq_basis_row_meta(int64_t ld, const int64_t* data_offsets,
                                    const int32_t* fock_block_offsets,
                                    const int32_t* atomic_numbers, const int32_t* rows,
                                    const int32_t* cols, int64_t num_rows,
                                    const int32_t* pair_kind, int maxe, int32_t* row_meta,
                                    void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && num_rows < (int64_t(1) << 31), "bad number of rows");
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(fock_block_offsets && atomic_numbers && rows && cols && pair_kind && row_meta,
                "null pointer");
  MALOQ_REQUIRE(data_offsets || (ld > 0 && ld < (int64_t(1) << 23)),
                "dense Fock row stride %lld out of range", static_cast<long long>(ld));
  MALOQ_REQUIRE(maxe > 0 && maxe <= 65535, "largest block size %d out of range", maxe);
  MALOQ_REQUIRE((reinterpret_cast<uintptr_t>(row_meta) & 15) == 0, "row_meta must be 16-byte aligned");
  const int64_t groups = (num_rows + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(bt::row_meta_kernel, dim3(static_cast<unsigned>(groups)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), num_rows, data_offsets ? 0 : ld,
                     data_offsets, fock_block_offsets, atomic_numbers, rows, cols, pair_kind,
                     maxe, reinterpret_cast<int4*>(row_meta));
  return check_launch("row plan");
}

extern "C" int maloq_fock_to_irreps(const float* fock, int64_t ld, const int32_t* row_meta,
                                    int64_t num_rows, const int32_t* slots, int maxe,
                                    const uint32_t* kind_blocks, float* out,
                                    const int32_t* perm_out, int t, int nblocks,
                                    const int32_t* blocks, const float* w, const int32_t* sched,
                                    int ngroups, int group_cols, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0, "bad sizes");
  if (int rc = check_tables(t, nblocks, blocks, w, sched, ngroups, group_cols)) return rc;
  if (int rc = check_perms(ngroups, nullptr, perm_out)) return rc;
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(out, "null pointer");
  bt::Args a = base_args(num_rows, t, nblocks, blocks, w, sched, ngroups, group_cols);
  if (int rc = set_fock_side(a, const_cast<float*>(fock), ld, row_meta, slots, maxe, kind_blocks))
    return rc;
  a.out = out;
  a.perm_out = perm_out;
  return launch_transform<bt::FOCK, bt::ROWS>(a, stream, "fock -> irreps");
}

extern "C" int maloq_irreps_to_fock(const float* irreps, const int32_t* perm_in, float* fock,
                                    int64_t ld, const int32_t* row_meta, int64_t num_rows,
                                    const int32_t* slots, int maxe,
                                    const uint32_t* kind_blocks, int t, int nblocks,
                                    const int32_t* blocks, const float* w, const int32_t* sched,
                                    int ngroups, int group_cols, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0, "bad sizes");
  if (int rc = check_tables(t, nblocks, blocks, w, sched, ngroups, group_cols)) return rc;
  if (int rc = check_perms(ngroups, perm_in, nullptr)) return rc;
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(irreps, "null pointer");
  bt::Args a = base_args(num_rows, t, nblocks, blocks, w, sched, ngroups, group_cols);
  if (int rc = set_fock_side(a, fock, ld, row_meta, slots, maxe, kind_blocks)) return rc;
  a.in = irreps;
  a.perm_in = perm_in;
  return launch_transform<bt::ROWS, bt::FOCK>(a, stream, "irreps -> fock");
}

extern "C" int maloq_fock_to_irreps_pairs(const float* fock, int64_t ld, const int64_t* data_offsets,
                                          const int32_t* fock_block_offsets, const int32_t* atomic_numbers,
                                          const int32_t* rows, const int32_t* cols, int64_t num_rows,
                                          const int32_t* pair_kind, const int32_t* slots, int maxe,
                                          const uint32_t* kind_blocks, float* out, const int32_t* perm_out,
                                          int t, int nblocks, const int32_t* blocks, const float* w,
                                          const int32_t* sched, int ngroups, int group_cols, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0, "bad sizes");
  if (int rc = check_tables(t, nblocks, blocks, w, sched, ngroups, group_cols)) return rc;
  if (int rc = check_perms(ngroups, nullptr, perm_out)) return rc;
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(out, "null pointer");
  bt::Args a = base_args(num_rows, t, nblocks, blocks, w, sched, ngroups, group_cols);
  if (int rc = set_fock_pairs(a, const_cast<float*>(fock), ld, data_offsets, fock_block_offsets, atomic_numbers,
                              rows, cols, num_rows, pair_kind, slots, maxe, kind_blocks))
    return rc;
  a.out = out;
  a.perm_out = perm_out;
  return launch_transform<bt::FOCK, bt::ROWS, true>(a, stream, "fock -> irreps (pair list)");
}

extern "C" int maloq_irreps_to_fock_pairs(const float* irreps, const int32_t* perm_in, float* fock, int64_t ld,
                                          const int64_t* data_offsets, const int32_t* fock_block_offsets,
                                          const int32_t* atomic_numbers, const int32_t* rows,
                                          const int32_t* cols, int64_t num_rows, const int32_t* pair_kind,
                                          const int32_t* slots, int maxe, const uint32_t* kind_blocks,
                                          int t, int nblocks, const int32_t* blocks, const float* w,
                                          const int32_t* sched, int ngroups, int group_cols, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0, "bad sizes");
  if (int rc = check_tables(t, nblocks, blocks, w, sched, ngroups, group_cols)) return rc;
  if (int rc = check_perms(ngroups, perm_in, nullptr)) return rc;
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(irreps, "null pointer");
  bt::Args a = base_args(num_rows, t, nblocks, blocks, w, sched, ngroups, group_cols);
  if (int rc = set_fock_pairs(a, fock, ld, data_offsets, fock_block_offsets, atomic_numbers, rows, cols, num_rows,
                              pair_kind, slots, maxe, kind_blocks))
    return rc;
  a.in = irreps;
  a.perm_in = perm_in;
  return launch_transform<bt::ROWS, bt::FOCK, true>(a, stream, "irreps -> fock (pair list)");
}

extern "C" int maloq_basis_cg_block(int program, float* w, int n) {
  MALOQ_REQUIRE(program >= 0 && program < cg::kPrograms, "CG program %d outside 0..%d", program,
                cg::kPrograms - 1);
  const int l1 = (program >> 2) & 3, l2 = program & 3;
  const int size = (2 * l1 + 1) * (2 * l2 + 1);
  MALOQ_REQUIRE(w != nullptr && n == size, "CG program %d is %d x %d (got n = %d)", program, size, size, n);
  for (int i = 0; i < size * size; ++i) w[i] = 0.f;
  for (int e = cg::kFirst[program]; e < cg::kFirst[program + 1]; ++e) w[cg::kRow[e] * size + cg::kCol[e]] = cg::kVal[e];
  return MALOQ_OK;
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
