// Weight gradients of the SO(2) linear (gfx950).
//
// bf16: dw_tr_kernel.  A workgroup owns a 256 x 256 tile of one C_g and a
// contiguous range of edges (split-K); each of its 4 waves a 128 x 128
// quarter (4 x 4 MFMA 32x32 tiles, accumulators in AGPRs).  Both operands are
// copied in their natural [edge][channel] layout straight from global memory
// into a 4-stage LDS ring (global_load_lds, 16-byte chunks XOR-swizzled by
// edge row so that the transposed reads are free of bank conflicts), 32 edges
// per stage, three stages in flight; MFMA operands (8 consecutive edges of one
// channel per lane) come from ds_read_b64_tr_b16, which transposes 4x4 blocks
// of 16-bit elements across each 16-lane group.
// fp32: dw_kernel below (register transposes).
//
// With Y_e the rotated, radially scaled input rows and dZ_e the rotated output
// gradient rows of edge e (both saved in m-major order [E, d', C] by the
// fused kernels), the gradient of every |m| group is a GEMM with the edges as
// the reduction axis:  C_g = sum_e dZ_g(e)^T Y_g(e), g = 0..mmax.
//
// Tiling.  A workgroup (4 waves) owns a 128 x 128 tile of one C_g and a
// contiguous edge range (split-K).  Each K step covers KE edges (64 bf16 /
// 16 fp32): every thread loads one VEC x VEC block (VEC edges x VEC columns,
// one 16-byte load per edge, coalesced along the columns), transposes it in
// registers and writes VEC 16-byte rows straight into MFMA fragment order, so
// both operands are K(edge)-contiguous per lane.  Loads for step s+1 are
// issued before the MFMAs of step s and land in the other LDS buffer (one
// barrier per step).  Each wave computes a 64 x 64 sub-tile (2 x 2 MFMA
// tiles of 32 x 32).  Partial tiles are summed in split order by
// dw_reduce_kernel, which also folds the +-m quadrants of C_m back into the
// reference layout of so2_m_conv.fc.weight:
//   dWr = C[+,+] + C[-,-],   dWi = C[-,+] - C[+,-]      (so2_layers.py:61-67).
// Deterministic: no atomics.
#include "message_impl.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace msg {

constexpr int MAXG = 8;
constexpr int DW_T = 128;  // output tile edge

struct DwArgs {
  const void* dz;       // [E, dpz, C_out]
  const void* y;        // [E, dpy, C_in]
  int64_t E;
  int dpz, dpy, C_out, C_in, ngroups, splits;
  // group g: dz rows [row0z, row0z + rowsz) x y rows [row0y, row0y + rowsy)
  int row0z[MAXG], rowsz[MAXG], row0y[MAXG], rowsy[MAXG];
  int gate;                  // last group: dL/dgate rows x m = 0 rows
  int ntk[MAXG];             // DW_T-wide tiles along k (= rows * C_in)
  int64_t tile0[MAXG + 1];   // cumulative tile counts
  int64_t goff[MAXG + 1];    // element offset of group g in one split's partials
  int64_t e_per_split;       // multiple of the K step
  float* part;               // [splits, goff[ngroups]]
};

template <class TM>
struct DwCfg {
  static constexpr int VEC = TM::VEC;            // elements per 16-byte row
  static constexpr int KC = TM::KC;              // edges per MFMA fragment
  static constexpr int KE = VEC * VEC * 256 / (2 * DW_T);  // edges per K step (1 block per thread)
  static constexpr int NSUB = KE / KC;           // fragment columns per step
  static constexpr int FRAGS = (DW_T / 32) * NSUB;  // fragments per operand per step
  static constexpr int STAGE = 2 * FRAGS * FRAG;    // A + B bytes per step
  // fp32: four waves per SIMD (the accumulators then live in VGPRs, 118 in
  // all, no spills); bf16 keeps its registers (it runs only where the
  // transpose-read kernel cannot)
  static constexpr int MIN_WAVES = TM::VEC == 4 ? 4 : 1;
};

// Transposes a VEC x VEC block held as VEC rows of 16 bytes (row = edge,
// VEC column elements) into VEC rows of VEC edges (row = column).
__device__ __forceinline__ void transpose_block(const uint4 (&in)[8], uint4 (&out)[8], BF16) {
  // 16-bit elements: word w of out[c] = (in[2w] elem c) | (in[2w+1] elem c) << 16
  const uint32_t* iw = reinterpret_cast<const uint32_t*>(in);
  uint32_t* ow = reinterpret_cast<uint32_t*>(out);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t lo = iw[(2 * w) * 4 + (c >> 1)], hi = iw[(2 * w + 1) * 4 + (c >> 1)];
      // v_perm_b32 selector: bytes of hi are 4..7, bytes of lo 0..3
      const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
      ow[c * 4 + w] = __builtin_amdgcn_perm(hi, lo, sel);
    }
  }
}
__device__ __forceinline__ void transpose_block(const uint4 (&in)[4], uint4 (&out)[4], F32) {
  const uint32_t* iw = reinterpret_cast<const uint32_t*>(in);
  uint32_t* ow = reinterpret_cast<uint32_t*>(out);
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) ow[c * 4 + e] = iw[e * 4 + c];
}

template <class TM>
__global__ __launch_bounds__(256, DwCfg<TM>::MIN_WAVES) void dw_kernel(DwArgs a) {
  using Cfg = DwCfg<TM>;
  constexpr int VEC = Cfg::VEC, KE = Cfg::KE, NSUB = Cfg::NSUB;
  __shared__ alignas(16) char smem[2 * Cfg::STAGE];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t ntiles = a.tile0[a.ngroups];
  // XCD-aware order, as in dw_tr_kernel: the tiles of one split (which read
  // the same dZ and Y rows) run on one XCD and share its L2
  const int64_t per = gridDim.x >> 3;
  const int64_t wid = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (wid >= ntiles * a.splits) return;  // whole workgroup, before any barrier
  const int64_t split = wid / ntiles;
  const int64_t t = wid % ntiles;
  int g = 0;
  while (g + 1 < a.ngroups && t >= a.tile0[g + 1]) ++g;
  const int64_t lt = t - a.tile0[g];
  const int tn = static_cast<int>(lt / a.ntk[g]), tk = static_cast<int>(lt % a.ntk[g]);
  const int Ng = a.rowsz[g] * a.C_out, Kg = a.rowsy[g] * a.C_in;
  const int64_t eb = split * a.e_per_split;
  const int64_t ee = (eb + a.e_per_split) < a.E ? (eb + a.e_per_split) : a.E;

  // this thread's block: operand (0 = dZ -> A, 1 = Y -> B), column group, edge group
  const int op = tid >> 7;
  const int bi = tid & 127;
  const int cg = bi % (DW_T / VEC), eg = bi / (DW_T / VEC);
  const int C = op ? a.C_in : a.C_out;
  const int col = (op ? tk : tn) * DW_T + cg * VEC;   // first column of the block in C_g
  const int lim = op ? Kg : Ng;
  const typename TM::raw* src = reinterpret_cast<const typename TM::raw*>(op ? a.y : a.dz);
  int64_t coladdr = -1;  // element offset of (edge 0, col) or -1 if the block is outside the tile
  if (col < lim) coladdr = static_cast<int64_t>((op ? a.row0y[g] : a.row0z[g]) + col / C) * C + col % C;
  const int64_t estride = static_cast<int64_t>(op ? a.dpy : a.dpz) * C;
  // LDS destination: fragment (col tile, k-substep), row = column within the tile
  const int cl = cg * VEC;  // column within the 128 tile
  const int e_in = eg * VEC;
  const int frag = op * Cfg::FRAGS + (cl >> 5) * NSUB + e_in / TM::KC;
  const int lds_off = frag * FRAG + frag_off<TM>(cl & 31, e_in % TM::KC);  // + c * row pitch below

  uint4 regs[VEC];
  auto load = [&](int64_t e0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int64_t e = e0 + e_in + v;
      regs[v] = make_uint4(0u, 0u, 0u, 0u);
      if (coladdr >= 0 && e < ee) regs[v] = *reinterpret_cast<const uint4*>(src + e * estride + coladdr);
    }
  };
  auto store = [&](int buf) {
    uint4 tr[VEC];
    transpose_block(regs, tr, TM{});
    char* base = smem + buf * Cfg::STAGE + lds_off;
#pragma unroll
    for (int c = 0; c < VEC; ++c)
      *reinterpret_cast<uint4*>(base + frag_off<TM>(c, 0) - frag_off<TM>(0, 0)) = tr[c];
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int wn = wave >> 1, wk = wave & 1;
  const int64_t nsteps = ee > eb ? (ee - eb + KE - 1) / KE : 0;
  if (nsteps > 0) {
    load(eb);
    store(0);
  }
  __syncthreads();
  for (int64_t s = 0; s < nsteps; ++s) {
    const bool more = s + 1 < nsteps;
    if (more) load(eb + (s + 1) * KE);
    const char* A = smem + (s & 1) * Cfg::STAGE;
    const char* B = A + Cfg::FRAGS * FRAG;
#pragma unroll
    for (int ks = 0; ks < NSUB; ++ks) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          mma(acc[i][j], A + ((2 * wn + i) * NSUB + ks) * FRAG, B + ((2 * wk + j) * NSUB + ks) * FRAG,
              lane, TM{});
    }
    if (more) store((s + 1) & 1);
    __syncthreads();
  }
  float* out = a.part + split * a.goff[a.ngroups] + a.goff[g];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int k = tk * DW_T + (2 * wk + j) * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = tn * DW_T + (2 * wn + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < Ng && k < Kg) out[static_cast<int64_t>(n) * Kg + k] = acc[i][j][r];
      }
  }
}

namespace trdw {
constexpr int T = 256;                  // output tile edge
constexpr int KE = 32;                  // edges per K step (two 16-edge MFMA k-substeps)
constexpr int NS = 4;                   // LDS ring stages
constexpr int PITCH = T * 2;            // bytes per staged edge row (bf16)
constexpr int TILE = KE * PITCH;        // 16 KB per operand per stage
constexpr int CHUNK = NS * KE;          // 128: split and padding granularity (edges)
}  // namespace trdw

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short v4s16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s16 lds_v4s16;

// Transposed fragment read: 4 edges x 1 channel of a staged tile (see above).
__device__ __forceinline__ v4s16 tr_read(const char* lds) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4s16*)((__attribute__((address_space(3))) const char*)lds));
}

// One K step on stage (sa, sb): 2 k-substeps x 4 x 4 MFMAs per wave.
// la[t], lb[t]: this lane's byte offsets inside the operand tiles for column
// tile t (row, swizzled chunk and wave-half part); the per-(ks, r) offsets are
// compile-time.
__device__ __forceinline__ void trdw_step(f32x16 (&acc)[4][4], const char* sa, const char* sb,
                                          const int (&la)[4], const int (&lb)[4]) {
  using namespace trdw;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    bf16x8 af[4], bfr[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      // rows 16 ks + {0, 4} + (lane part) of column tile t
      v4s16 a0 = tr_read(sa + la[t] + (ks * 16 + 0) * PITCH);
      v4s16 a1 = tr_read(sa + la[t] + (ks * 16 + 4) * PITCH);
      v4s16 b0 = tr_read(sb + lb[t] + (ks * 16 + 0) * PITCH);
      v4s16 b1 = tr_read(sb + lb[t] + (ks * 16 + 4) * PITCH);
      af[t] = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
      bfr[t] = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
  }
}

__global__ __launch_bounds__(256, 1) void dw_tr_kernel(DwArgs a) {
  using namespace trdw;
  __shared__ alignas(16) char A0[TILE], B0[TILE], A1[TILE], B1[TILE], A2[TILE], B2[TILE],
      A3[TILE], B3[TILE];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t ntiles = a.tile0[a.ngroups];
  // XCD-aware order: workgroups go round-robin over the 8 XCDs, so work item
  // (xcd * per + i) runs as workgroup 8 i + xcd; consecutive work items (the
  // tiles of one split, which share operand rows) then share one XCD's L2.
  // The grid is padded to a multiple of 8; the padding exits at once.
  const int64_t per = gridDim.x >> 3;
  const int64_t wid = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (wid >= ntiles * a.splits) return;  // whole workgroup, before any barrier
  const int64_t split = wid / ntiles;
  const int64_t t = wid % ntiles;
  int g = 0;
  while (g + 1 < a.ngroups && t >= a.tile0[g + 1]) ++g;
  const int64_t lt = t - a.tile0[g];
  const int tn = static_cast<int>(lt / a.ntk[g]), tk = static_cast<int>(lt % a.ntk[g]);
  const int Ng = a.rowsz[g] * a.C_out, Kg = a.rowsy[g] * a.C_in;
  const int64_t eb = split * a.e_per_split;
  const int64_t epad = (a.E + CHUNK - 1) / CHUNK * CHUNK;
  const int64_t ee = (eb + a.e_per_split) < epad ? (eb + a.e_per_split) : epad;
  const int nsteps = ee > eb ? static_cast<int>((ee - eb) / KE) : 0;  // a multiple of NS

  // DMA: wave w copies chunks p = (4 w + j) 64 + lane of each operand tile
  // (row r = p / 32, slot p % 32), loading global chunk (slot ^ (r & 7)).
  const uint16_t* za = reinterpret_cast<const uint16_t*>(a.dz) +
                       static_cast<int64_t>(a.row0z[g]) * a.C_out + static_cast<int64_t>(tn) * T;
  const uint16_t* yb = reinterpret_cast<const uint16_t*>(a.y) +
                       static_cast<int64_t>(a.row0y[g]) * a.C_in + static_cast<int64_t>(tk) * T;
  const int64_t sa_e = static_cast<int64_t>(a.dpz) * a.C_out, sb_e = static_cast<int64_t>(a.dpy) * a.C_in;
  int dr[4], dc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int p = (wave * 4 + j) * 64 + lane;
    dr[j] = p >> 5;
    dc[j] = ((p & 31) ^ ((dr[j] & 3) << 2)) * 8;  // LDS chunk s of row r holds chunk s ^ 4 (r % 4)
  }
  // The copies are issued by inline asm, invisible to the compiler's wait
  // insertion (which would otherwise drain the ring before LDS reads it cannot
  // tell apart); the explicit vmcnt/barrier of each step orders them.
  auto dma = [&](char* da, char* db, int step) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int64_t e = eb + static_cast<int64_t>(step) * KE + dr[j];
      e = e < epad ? e : epad - 1;  // steps past the range: in-bounds, never read
      const uint16_t* ga = za + e * sa_e + dc[j];
      const uint16_t* gb = yb + e * sb_e + dc[j];
      const unsigned la_s = __builtin_amdgcn_readfirstlane(
          static_cast<unsigned>(reinterpret_cast<size_t>((__attribute__((address_space(3))) char*)(da + (wave * 4 + j) * 1024))));
      const unsigned lb_s = __builtin_amdgcn_readfirstlane(
          static_cast<unsigned>(reinterpret_cast<size_t>((__attribute__((address_space(3))) char*)(db + (wave * 4 + j) * 1024))));
      asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(ga), "s"(la_s) : "memory", "m0");
      asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gb), "s"(lb_s) : "memory", "m0");
    }
  };
  // transposed reads: lane (g16 = lane/16, a = lane%4, kk = lane/4%4) addresses row
  // 8 (g16/2) + 4 r + kk + 16 ks, column 32 t + 16 (g16%2) + 4 a of its wave's half,
  // i.e. 16-byte chunk c = 4 t + 2 (g16%2) + a/2, stored at chunk c ^ 4 kk: the 4
  // rows x 4 chunks of one read land in 16 distinct chunks (no bank conflicts)
  const int g16 = lane >> 4, aa = lane & 3, kk = (lane >> 2) & 3;
  const int lrow = (8 * (g16 >> 1) + kk) * PITCH + (2 * (g16 & 1) + (aa >> 1)) * 16 + (aa & 1) * 8;
  const int wm = wave >> 1, wn = wave & 1;
  int la[4], lb[4];  // the wave's 128-column half = 16 chunks
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    la[t] = lrow + wm * 256 + 64 * (t ^ kk);
    lb[t] = lrow + wn * 256 + 64 * (t ^ kk);
  }

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  dma(A0, B0, 0);
  dma(A1, B1, 1);
  dma(A2, B2, 2);
  for (int s = 0; s < nsteps; s += NS) {
    // each step: this wave's copies of the step done (two later steps in flight),
    // then all waves' (barrier); the stage refilled was read one step earlier
#define MALOQ_TRDW_STEP(SA, SB, NA, NB, K)                                           \
    asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");     \
    dma(NA, NB, s + K + 3);                                                         \
    trdw_step(acc, SA, SB, la, lb);
    MALOQ_TRDW_STEP(A0, B0, A3, B3, 0)
    MALOQ_TRDW_STEP(A1, B1, A0, B0, 1)
    MALOQ_TRDW_STEP(A2, B2, A1, B1, 2)
    MALOQ_TRDW_STEP(A3, B3, A2, B2, 3)
#undef MALOQ_TRDW_STEP
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy left in flight at exit

  float* out = a.part + split * a.goff[a.ngroups] + a.goff[g];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = tk * T + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = tn * T + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < Ng && n < Kg) out[static_cast<int64_t>(m) * Kg + n] = acc[i][j][r];
      }
    }
}

// One thread per element of the reference-layout gradients:
// dW0 [(gate ? L : 0) C_out + (L+1) C_out, (L+1) C_in] (gate rows first, as in
// fc_m0, so2_layers.py:112-115), then dW_m [2 (L-m+1) C_out, (L-m+1) C_in].
// Destinations of the m >= 1 gradients (a kernel argument by value).
struct DwOut {
  float* m[MAXG];
};

__global__ void dw_reduce_kernel(DwArgs a, int lmax, float* __restrict__ dw0, DwOut dwm) {
  const int g = blockIdx.y;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t Kg = static_cast<int64_t>(a.rowsy[g]) * a.C_in;
  const int64_t stride = a.goff[a.ngroups];
  auto C = [&](int64_t n, int64_t k) {
    const float* p = a.part + a.goff[g] + n * Kg + k;
    float s = 0.f;
    for (int sp = 0; sp < a.splits; ++sp) s += p[sp * stride];
    return s;
  };
  const bool gate_group = a.gate && g == a.ngroups - 1;
  if (g == 0 || gate_group) {
    const int64_t Ng = static_cast<int64_t>(a.rowsz[g]) * a.C_out;
    if (idx >= Ng * Kg) return;
    float* d = dw0 + ((g == 0 && a.gate) ? static_cast<int64_t>(lmax) * a.C_out * Kg : 0);
    d[idx] = C(idx / Kg, idx % Kg);
    return;
  }
  const int m = g;
  const int64_t nr = lmax - m + 1;  // rows per sign
  const int64_t ho = nr * a.C_out, ki_n = nr * a.C_in;
  if (idx >= 2 * ho * ki_n) return;
  const int64_t r = idx / ki_n, ki = idx % ki_n;
  float v;
  if (r < ho) {  // dWr[ko][ki] = C[+ko][+ki] + C[-ko][-ki]
    v = C(r, ki) + C(ho + r, ki_n + ki);
  } else {       // dWi[ko][ki] = C[-ko][+ki] - C[+ko][-ki]
    const int64_t ko = r - ho;
    v = C(ho + ko, ki) - C(ko, ki_n + ki);
  }
  float* dst = dwm.m[m - 1];
  dst[idx] = v;
}

}  // namespace msg
}  // namespace maloq

using namespace maloq;
using namespace maloq::msg;

// tile: output tile edge (128 for dw_kernel, 256 for dw_tr_kernel); gran:
// split boundaries are multiples of this many edges.
// Groups: m = 0 (rows 0..L of both), +-m for m = 1..mmax (stacked), and for a
// gated block dz's gate rows (after the kept rows) against y's m = 0 rows.
static int dw_setup(DwArgs& a, int lmax, int mmax, int gate, int64_t E, int c_out, int c_in,
                    int splits, int tile, int gran) {
  MALOQ_REQUIRE(mmax >= 0 && mmax + 2 <= MAXG && mmax <= lmax, "mmax out of range for the weight gradient");
  MALOQ_REQUIRE(splits >= 1 && splits <= 64, "splits out of range");
  a.E = E;
  a.C_out = c_out;
  a.C_in = c_in;
  a.gate = gate ? 1 : 0;
  a.ngroups = mmax + 1 + a.gate;
  a.splits = splits;
  int row = 0;
  for (int g = 0; g <= mmax; ++g) {
    const int r = (g == 0) ? (lmax + 1) : 2 * (lmax - g + 1);
    a.row0z[g] = a.row0y[g] = row;
    a.rowsz[g] = a.rowsy[g] = r;
    row += r;
  }
  a.dpy = row;
  a.dpz = row + (gate ? lmax : 0);
  if (gate) {
    a.row0z[mmax + 1] = row;
    a.rowsz[mmax + 1] = lmax;
    a.row0y[mmax + 1] = 0;
    a.rowsy[mmax + 1] = lmax + 1;
  }
  a.tile0[0] = 0;
  a.goff[0] = 0;
  for (int g = 0; g < a.ngroups; ++g) {
    const int64_t Ng = static_cast<int64_t>(a.rowsz[g]) * c_out, Kg = static_cast<int64_t>(a.rowsy[g]) * c_in;
    a.ntk[g] = static_cast<int>((Kg + tile - 1) / tile);
    a.tile0[g + 1] = a.tile0[g] + ((Ng + tile - 1) / tile) * a.ntk[g];
    a.goff[g + 1] = a.goff[g] + Ng * Kg;
  }
  a.e_per_split = ((E + splits - 1) / splits + gran - 1) / gran * gran;
  return MALOQ_OK;
}

// Rows the bf16 weight gradient reads from dz / y: the edges rounded up to a
// whole number of 128-edge chunks, plus one row (tiles that end past a row's
// last column read into the next row).  Rows from num_edges on must be zero.
static int64_t dw_rows(int64_t E) { return (E + trdw::CHUNK - 1) / trdw::CHUNK * trdw::CHUNK + 1; }

extern "C" int64_t maloq_message_edge_rows(int64_t num_edges) {
  return num_edges < 0 ? -1 : dw_rows(num_edges);
}

extern "C" int64_t maloq_message_dw_partials_floats(int lmax, int mmax, int gate, int c_out, int c_in,
                                                    int splits) {
  DwArgs a{};
  if (dw_setup(a, lmax, mmax, gate, 0, c_out, c_in, splits, DW_T, 64)) return -1;
  int64_t n = a.goff[a.ngroups] * splits;
  // the bf16 kernel's 256-wide tiles give the same group sizes (goff does not depend on the tile)
  return n;
}

extern "C" int maloq_message_dw(int dtype, int lmax, int mmax, int gate, const void* dz, const void* y,
                                int64_t num_edges, int c_out, int c_in, int splits,
                                float* partials, float* dw0, float* const* dwm,
                                void* stream) {
  MALOQ_REQUIRE(dtype == 0 || dtype == 1, "dtype must be 0 (fp32) or 1 (bf16)");
  MALOQ_REQUIRE(num_edges >= 0, "num_edges < 0");
  MALOQ_REQUIRE(c_out > 0 && c_in > 0, "bad channels");
  DwArgs a{};
  int rc = dw_setup(a, lmax, mmax, gate, num_edges, c_out, c_in, splits, DW_T, 64);
  if (rc) return rc;
  // bf16 rows of at least one tile (a tile ending past a row's last column
  // reads into the next row): the transpose-read kernel; else dw_kernel.
  const bool tr = dtype == 1 && c_out % 8 == 0 && c_in % 8 == 0 &&
                  static_cast<int64_t>(a.dpz) * c_out >= trdw::T && static_cast<int64_t>(a.dpy) * c_in >= trdw::T;
  if (tr) {
    rc = dw_setup(a, lmax, mmax, gate, num_edges, c_out, c_in, splits, trdw::T, trdw::CHUNK);
    if (rc) return rc;
  }
  MALOQ_REQUIRE(partials && dw0, "null pointer");
  DwOut outm{};
  MALOQ_REQUIRE(mmax == 0 || dwm, "dwm is null");
  for (int m = 1; m <= mmax; ++m) {
    MALOQ_REQUIRE(dwm[m - 1], "dwm[%d] is null", m - 1);
    outm.m[m - 1] = dwm[m - 1];
  }
  MALOQ_REQUIRE(num_edges == 0 || (dz && y), "null pointer");
  a.dz = dz;
  a.y = y;
  a.part = partials;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // both kernels map workgroups to work items per XCD (grid a multiple of 8)
  const int64_t grid = (a.tile0[a.ngroups] * splits + 7) / 8 * 8;
  MALOQ_REQUIRE(grid < (int64_t(1) << 31), "grid too large");
  if (tr)
    hipLaunchKernelGGL(dw_tr_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, a);
  else if (dtype == 1)
    hipLaunchKernelGGL(dw_kernel<BF16>, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(dw_kernel<F32>, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, a);
  rc = check_launch("dw_kernel");
  if (rc) return rc;
  int64_t maxel = 0;
  for (int g = 0; g < a.ngroups; ++g) {
    const int64_t el = static_cast<int64_t>(a.rowsz[g]) * c_out * a.rowsy[g] * c_in;
    maxel = el > maxel ? el : maxel;
  }
  hipLaunchKernelGGL(dw_reduce_kernel, dim3(static_cast<unsigned>((maxel + 255) / 256), a.ngroups),
                     dim3(256), 0, s, a, lmax, dw0, outm);
  return check_launch("dw_reduce_kernel");
}
