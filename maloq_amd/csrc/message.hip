// C ABI of the fused message block (forward and input gradient) and the
// partial-segment fixup.  The kernels themselves are in message_impl.h and
// are instantiated per lmax in message_l{2,4,6}.hip.
#include <mutex>

#include "message_launch.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace msg {

// Node outputs of segments cut by tile boundaries (summed in tile order) and
// of empty segments (zero).  seg_ptr: CSR of the segment ids over edges.  A
// workgroup per node, 16-byte columns (row_elems a multiple of 4); the
// workgroups of nodes the main kernel wrote in full exit at once.
__global__ __launch_bounds__(256) void message_fixup_kernel(const int64_t* __restrict__ seg_ptr,
                                                            const float* __restrict__ part,
                                                            float* __restrict__ out, int64_t row_elems,
                                                            int TE) {
  const int64_t node = blockIdx.x;
  const int64_t s0 = seg_ptr[node], s1 = seg_ptr[node + 1];
  float4* o = reinterpret_cast<float4*>(out + node * row_elems);
  const int64_t n4 = row_elems / 4;
  if (s1 == s0) {
    for (int64_t c = threadIdx.x; c < n4; c += blockDim.x) o[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    return;
  }
  const int64_t t0 = s0 / TE, t1 = (s1 - 1) / TE;
  if (t0 == t1) return;  // written by the main kernel
  const float4* first = reinterpret_cast<const float4*>(part + ((t0 * 2) + ((s0 == t0 * TE) ? 0 : 1)) * row_elems);
  for (int64_t c = threadIdx.x; c < n4; c += blockDim.x) {
    float4 sum = first[c];
    for (int64_t t = t0 + 1; t <= t1; ++t) {
      const float4 v = reinterpret_cast<const float4*>(part + (t * 2) * row_elems)[c];
      sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
    }
    o[c] = sum;
  }
}

// Packed B fragments per output-channel block: for every kernel-input degree
// li and K step, per output degree lo: g0, [gate], (Wr, Wi) for m <= min(mmax, li, lo).
// The gate fragment is there for lo >= 1 in the forward and for li >= 1 in the
// input gradient: the same count either way.
static int64_t frags_per_cb(int lmax, int mmax, int gate, int c_k, int kc) {
  int64_t total = 0;
  for (int li = 0; li <= lmax; ++li) {
    int nb = 0;
    for (int lo = 0; lo <= lmax; ++lo) {
      int mm = mmax < li ? mmax : li;
      mm = mm < lo ? mm : lo;
      nb += 1 + ((gate && lo >= 1) ? 1 : 0) + 2 * mm;
    }
    total += static_cast<int64_t>(nb) * (c_k / kc);
  }
  return total;
}

static int fixup(const int64_t* seg_ptr, int64_t nseg, const float* part, float* out,
                 int64_t row_elems, int TE, hipStream_t s) {
  if (nseg == 0) return MALOQ_OK;
  MALOQ_REQUIRE(row_elems % 4 == 0, "row width must be a multiple of 4");
  MALOQ_REQUIRE(((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(part)) & 15) == 0,
                "output and partials must be 16-byte aligned");
  MALOQ_REQUIRE(nseg < (int64_t(1) << 31), "too many segments");
  hipLaunchKernelGGL(message_fixup_kernel, dim3(static_cast<unsigned>(nseg)), dim3(256), 0, s, seg_ptr, part,
                     out, row_elems, TE);
  return check_launch("message_fixup_kernel");
}

static int dispatch(int lmax, int mmax, int dtype, int gate, int mode, const Args& a,
                    hipStream_t s) {
  switch (lmax) {
    case 2: return launch_l2(mmax, dtype, gate, mode, a, s);
    case 4: return launch_l4(mmax, dtype, gate, mode, a, s);
    case 6: return launch_l6(mmax, dtype, gate, mode, a, s);
    default: break;
  }
  MALOQ_REQUIRE(false, "unsupported lmax %d (built: (lmax, mmax) in (2, 2), (4, 2), (4, 4), (6, 2), (6, 6))", lmax);
}

static int prep_dispatch(int lmax, int mmax, int dtype, int mode, const PrepArgs& a,
                         hipStream_t s) {
  switch (lmax) {
    case 2: return prep_l2(mmax, dtype, mode, a, s);
    case 4: return prep_l4(mmax, dtype, mode, a, s);
    case 6: return prep_l6(mmax, dtype, mode, a, s);
    default: break;
  }
  MALOQ_REQUIRE(false, "unsupported lmax %d (built: (lmax, mmax) in (2, 2), (4, 2), (4, 4), (6, 2), (6, 6))", lmax);
}

static int check_common(int dtype, int lmax, int mmax, int c_k, int c_n, int64_t E) {
  MALOQ_REQUIRE(dtype == 0 || dtype == 1, "dtype must be 0 (fp32) or 1 (bf16)");
  MALOQ_REQUIRE(lmax >= 0 && mmax >= 0 && mmax <= lmax, "bad lmax/mmax");
  const int kc = dtype == 1 ? BF16::KC : F32::KC;
  MALOQ_REQUIRE(c_k > 0 && c_k % kc == 0, "input channels must be a positive multiple of %d", kc);
  MALOQ_REQUIRE(c_n > 0 && c_n % CB == 0, "output channels must be a positive multiple of %d", CB);
  MALOQ_REQUIRE(E >= 0 && E < (int64_t(1) << 31), "edge count out of range");
  return MALOQ_OK;
}

static int kept_rows(int lmax, int mmax) {
  int r = lmax + 1;
  for (int m = 1; m <= mmax; ++m) r += 2 * (lmax - m + 1);
  return r;
}

// Floats per edge of the kept Wigner rows in the pair-major layout
// (PairLayout in message_impl.h): per degree l, (l+1) column pairs of
// 2 (1 + 2 min(mmax, l)) floats, each rounded up to a multiple of 4.
static int wigner_floats(int lmax, int mmax) {
  int s = 0;
  for (int l = 0; l <= lmax; ++l) s += (l + 1) * ((2 * (1 + 2 * (mmax < l ? mmax : l)) + 3) / 4 * 4);
  return s;
}

}  // namespace msg
}  // namespace maloq

using namespace maloq;
using namespace maloq::msg;

extern "C" int maloq_message_kept_rows(int lmax, int mmax) { return kept_rows(lmax, mmax); }

extern "C" int maloq_message_wigner_floats(int lmax, int mmax) { return wigner_floats(lmax, mmax); }

extern "C" int maloq_message_supported(int lmax, int mmax) {
  return (lmax == 2 && mmax == 2) || ((lmax == 4 || lmax == 6) && (mmax == 2 || mmax == lmax)) ? 1 : 0;
}

extern "C" int64_t maloq_message_partials_floats(int lmax, int gate, int64_t num_edges, int c_out) {
  const int64_t d = static_cast<int64_t>(lmax + 1) * (lmax + 1);
  const int64_t te = MIN_TILE_EDGES;  // sized for the smallest tile of any instantiation
  return ((num_edges + te - 1) / te) * 2 * d * c_out;
}

extern "C" int64_t maloq_message_wpack_bytes(int dtype, int lmax, int mmax, int gate, int c_k,
                                             int c_n) {
  const int kc = dtype == 1 ? BF16::KC : F32::KC;
  if (c_k % kc != 0 || c_n % CB != 0) return -1;
  return frags_per_cb(lmax, mmax, gate, c_k, kc) * (c_n / CB) * FRAG;
}

extern "C" int maloq_message_fwd(int dtype, int lmax, int mmax, int gate, const void* x, int c_in,
                                 const int32_t* src, const int32_t* dst, int64_t num_edges,
                                 const float* eulers, const void* rad, const void* wpack,
                                 const float* bias, const float* jd, float* out, int64_t num_nodes,
                                 int c_out, const int64_t* seg_ptr, float* partials, void* y_ws,
                                 void* r_ws, float* dk_ws, void* gate_ws, void* stream) {
  int rc = check_common(dtype, lmax, mmax, c_in, c_out, num_edges);
  if (rc) return rc;
  MALOQ_REQUIRE(num_nodes >= 0, "num_nodes < 0");
  MALOQ_REQUIRE(out && seg_ptr && jd && wpack, "null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t d = static_cast<int64_t>(lmax + 1) * (lmax + 1);
  if (num_edges > 0) {
    MALOQ_REQUIRE(x && src && dst && partials && y_ws && dk_ws, "null pointer");
    PrepArgs p{};
    p.x = x; p.gidx = src; p.eidx = nullptr; p.eulers = eulers; p.rad = rad; p.jd = jd;
    // without Euler triples dk_ws already holds the kept Wigner rows (maloq_message_wigner_rows)
    p.y = y_ws; p.r = r_ws; p.dk = dk_ws; p.build_d = eulers != nullptr; p.E = num_edges; p.C = c_in;
    rc = prep_dispatch(lmax, mmax, dtype, FWD, p, s);
    if (rc) return rc;
    Args a{};
    a.a_src = y_ws; a.dk = dk_ws; a.seg = dst; a.eidx = nullptr;
    a.wpack = static_cast<const char*>(wpack); a.bias = bias; a.out = out;
    a.part = partials; a.E = num_edges; a.C_k = c_in; a.C_n = c_out; a.n_cb = c_out / CB;
    a.extra = gate ? lmax * c_out : 0;
    a.ntiles = (num_edges + tile_edges(lmax, mmax, gate) - 1) / tile_edges(lmax, mmax, gate);
    const int kc = dtype == 1 ? BF16::KC : F32::KC;
    a.frags_per_cb = frags_per_cb(lmax, mmax, gate, c_in, kc);
    a.gsave = gate ? gate_ws : nullptr;
    rc = dispatch(lmax, mmax, dtype, gate, FWD, a, s);
    if (rc) return rc;
  }
  return fixup(seg_ptr, num_nodes, partials, out, d * c_out, tile_edges(lmax, mmax, gate), s);
}

// ------------------------------------------------- forward without allocation
// Workspace of maloq_message_fwd_noalloc: one file-scope device array per GPU
// (each device that loads the library holds its own copy until the process
// ends).  In host code the name `scratch` is only a stand-in symbol; its device
// address is looked up once per device with hipGetSymbolAddress and only that
// address is ever passed to a kernel.
static __device__ __align__(256) unsigned char scratch[MALOQ_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  MALOQ_REQUIRE(e == hipSuccess, "hipGetDevice: %s", hipGetErrorString(e));
  MALOQ_REQUIRE(dev >= 0 && dev < kMaxDevices, "device id %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    MALOQ_REQUIRE(e == hipSuccess && p != nullptr, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MALOQ_OK;
}

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }
}  // namespace

extern "C" int maloq_message_fwd_noalloc(int dtype, int lmax, int mmax, int gate, const void* x, int c_in,
                                         const int32_t* src, const int32_t* dst, int64_t num_edges,
                                         const float* eulers, const void* rad, const void* wpack,
                                         const float* bias, const float* jd, float* out, int64_t num_nodes,
                                         int c_out, const int64_t* seg_ptr, void* stream) {
  int rc = check_common(dtype, lmax, mmax, c_in, c_out, num_edges);
  if (rc) return rc;
  MALOQ_REQUIRE(maloq_message_supported(lmax, mmax), "no message kernels for lmax %d, mmax %d", lmax, mmax);
  MALOQ_REQUIRE(eulers != nullptr || num_edges == 0, "the no-allocation forward builds D from eulers");
  // workspace layout: partials | rotated rows y [E, d', c_in] | kept Wigner rows [E, WS]
  const int64_t part_b = align256(maloq_message_partials_floats(lmax, gate, num_edges, c_out) * 4);
  const int64_t y_b = align256(num_edges * kept_rows(lmax, mmax) * c_in * (dtype == 1 ? 2 : 4));
  const int64_t dk_b = align256(num_edges * wigner_floats(lmax, mmax) * 4);
  const int64_t need = part_b + y_b + dk_b;
  MALOQ_REQUIRE(need <= static_cast<int64_t>(MALOQ_NOALLOC_SCRATCH_BYTES),
                "maloq_message_fwd_noalloc: %lld edges need %lld bytes of workspace, the scratch array holds %lld",
                static_cast<long long>(num_edges), static_cast<long long>(need),
                static_cast<long long>(MALOQ_NOALLOC_SCRATCH_BYTES));
  void* base = nullptr;
  rc = scratch_ptr(&base);
  if (rc) return rc;
  char* b = static_cast<char*>(base);
  return maloq_message_fwd(dtype, lmax, mmax, gate, x, c_in, src, dst, num_edges, eulers, rad, wpack, bias, jd, out,
                           num_nodes, c_out, seg_ptr, reinterpret_cast<float*>(b), b + part_b, nullptr,
                           reinterpret_cast<float*>(b + part_b + y_b), nullptr, stream);
}

extern "C" int maloq_message_edgewise_fwd(int dtype, int lmax, int mmax, const void* x, int c_x,
                                          const int32_t* src, const int32_t* dst,
                                          const int32_t* seg_id, int64_t num_edges,
                                          const float* eulers, const void* rad, const void* wpack1,
                                          const float* bias1, int c_hidden, const void* wpack2,
                                          const float* bias2, const float* jd, float* out,
                                          int64_t num_nodes, int c_out, const int64_t* seg_ptr,
                                          float* partials, void* y_ws, void* r_ws, float* dk_ws,
                                          void* gate_ws, void* z_ws, const void* x_msg,
                                          const int32_t* msg_row, void* stream) {
  MALOQ_REQUIRE(c_x > 0 && c_x % 8 == 0, "node channels must be a positive multiple of 8");
  const int parts = x_msg ? 3 : 2;   // message parts: x[src], x[dst] [, x_msg[msg_row]]
  int rc = check_common(dtype, lmax, mmax, parts * c_x, c_hidden, num_edges);
  if (rc) return rc;
  rc = check_common(dtype, lmax, mmax, c_hidden, c_out, num_edges);
  if (rc) return rc;
  MALOQ_REQUIRE(num_nodes >= 0, "num_nodes < 0");
  MALOQ_REQUIRE(out && seg_ptr && jd && wpack1 && wpack2, "null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t d = static_cast<int64_t>(lmax + 1) * (lmax + 1);
  const int kc = dtype == 1 ? BF16::KC : F32::KC;
  if (num_edges > 0) {
    MALOQ_REQUIRE(x && src && dst && partials && y_ws && dk_ws && z_ws, "null pointer");
    MALOQ_REQUIRE(!x_msg || msg_row, "the edge message rows need msg_row");
    const int32_t* seg = seg_id ? seg_id : dst;
    // rotated message rows of cat(x[src], x[dst]) (radial scale applied) and the Wigner rows
    PrepArgs p{};
    p.x = x; p.gidx = src; p.gidx2 = dst; p.x3 = x_msg; p.gidx3 = msg_row; p.x_c = c_x;
    p.eidx = nullptr; p.eulers = eulers;
    p.rad = rad; p.jd = jd; p.y = y_ws; p.r = r_ws; p.dk = dk_ws; p.build_d = eulers != nullptr;
    p.E = num_edges; p.C = parts * c_x;
    rc = prep_dispatch(lmax, mmax, dtype, FWD, p, s);
    if (rc) return rc;
    // first convolution + gate, kept in the edge frame
    Args a{};
    a.a_src = y_ws; a.dk = dk_ws; a.seg = seg; a.eidx = nullptr;
    a.wpack = static_cast<const char*>(wpack1); a.bias = bias1; a.out = out; a.part = partials;
    a.E = num_edges; a.C_k = parts * c_x; a.C_n = c_hidden; a.n_cb = c_hidden / CB;
    a.extra = lmax * c_hidden;
    a.ntiles = (num_edges + tile_edges(lmax, mmax, 1, FWD_EDGE) - 1) / tile_edges(lmax, mmax, 1, FWD_EDGE);
    a.frags_per_cb = frags_per_cb(lmax, mmax, 1, parts * c_x, kc);
    a.gsave = gate_ws; a.zout = z_ws;
    rc = dispatch(lmax, mmax, dtype, 1, FWD_EDGE, a, s);
    if (rc) return rc;
    // second convolution, rotation back and segment sum
    Args b{};
    b.a_src = z_ws; b.dk = dk_ws; b.seg = seg; b.eidx = nullptr;
    b.wpack = static_cast<const char*>(wpack2); b.bias = bias2; b.out = out; b.part = partials;
    b.E = num_edges; b.C_k = c_hidden; b.C_n = c_out; b.n_cb = c_out / CB; b.extra = 0;
    b.ntiles = (num_edges + tile_edges(lmax, mmax, 0) - 1) / tile_edges(lmax, mmax, 0);
    b.frags_per_cb = frags_per_cb(lmax, mmax, 0, c_hidden, kc);
    rc = dispatch(lmax, mmax, dtype, 0, FWD, b, s);
    if (rc) return rc;
  }
  return fixup(seg_ptr, num_nodes, partials, out, d * c_out, tile_edges(lmax, mmax, 0), s);
}

extern "C" int maloq_message_edgewise_bwd_dx(
    int dtype, int lmax, int mmax, const float* grad_out, int c_x, const int32_t* dst,
    const int32_t* grad_row, const int32_t* src_sorted, const int32_t* edge_idx, int64_t num_edges, const float* dk,
    const void* rad, void* grad_rad, const void* r_saved, const void* gate_saved, const void* wpack1_t,
    int c_hidden, const void* wpack2_t, const float* jd, float* grad_x_src, float* grad_x_dst,
    int64_t num_nodes, const int64_t* seg_ptr, const int64_t* seg_ptr_src, float* partials,
    void* dz2_ws, void* dz1_ws, const int32_t* edge_seg, float* grad_x_msg, void* stream) {
  MALOQ_REQUIRE(c_x > 0 && c_x % CB == 0, "node channels must be a positive multiple of %d", CB);
  const int parts = grad_x_msg ? 3 : 2;
  int rc = check_common(dtype, lmax, mmax, c_x, c_hidden, num_edges);   // conv2 transposed
  if (rc) return rc;
  rc = check_common(dtype, lmax, mmax, c_hidden, parts * c_x, num_edges);   // conv1 transposed
  if (rc) return rc;
  MALOQ_REQUIRE(num_nodes >= 0, "num_nodes < 0");
  MALOQ_REQUIRE(grad_x_src && grad_x_dst && seg_ptr && seg_ptr_src && jd && wpack1_t && wpack2_t,
                "null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t d = static_cast<int64_t>(lmax + 1) * (lmax + 1);
  const int kc = dtype == 1 ? BF16::KC : F32::KC;
  if (num_edges > 0) {
    MALOQ_REQUIRE(grad_out && dst && src_sorted && edge_idx && dk && gate_saved && partials && dz2_ws &&
                  dz1_ws, "null pointer");
    MALOQ_REQUIRE(rad == nullptr || r_saved != nullptr, "the radial gradient needs the saved rows");
    MALOQ_REQUIRE(!grad_x_msg || edge_seg, "the edge message gradient needs edge_seg");
    // dL/d(conv2 output) in the edge frame: D_e grad_out[dst[e]]
    PrepArgs p{};
    p.x = grad_out; p.gidx = grad_row ? grad_row : dst; p.eidx = nullptr; p.jd = jd; p.y = dz2_ws;
    p.dk = const_cast<float*>(dk); p.build_d = 0; p.E = num_edges; p.C = c_x;
    rc = prep_dispatch(lmax, mmax, dtype, BWD_DX, p, s);
    if (rc) return rc;
    // conv2 transposed, rows kept in the edge frame and passed through the gate
    // backward: dL/dpre (kept rows) and dL/dgate rows of conv1
    Args b{};
    b.a_src = dz2_ws; b.dk = dk; b.seg = dst; b.eidx = nullptr;
    b.wpack = static_cast<const char*>(wpack2_t); b.out = grad_x_src; b.part = partials;
    b.E = num_edges; b.C_k = c_x; b.C_n = c_hidden; b.n_cb = c_hidden / CB;
    b.ntiles = (num_edges + tile_edges(lmax, mmax, 0) - 1) / tile_edges(lmax, mmax, 0);
    b.frags_per_cb = frags_per_cb(lmax, mmax, 0, c_x, kc);
    b.zout = dz1_ws; b.gsave = const_cast<void*>(gate_saved);
    rc = dispatch(lmax, mmax, dtype, 0, BWD_EDGE, b, s);
    if (rc) return rc;
    // conv1 transposed (gated input rows, radial gradient), one pass per message
    // part: the x[src] channels summed per source, the x[dst] channels per
    // destination, the edge message channels kept per edge (its own segment)
    for (int part = 0; part < parts; ++part) {
      Args a{};
      a.a_src = dz1_ws; a.dk = dk; a.seg = part == 0 ? src_sorted : (part == 1 ? dst : edge_seg);
      a.eidx = part == 0 ? edge_idx : nullptr;
      a.rad = rad; a.drad = grad_rad; a.rsave = r_saved;
      a.wpack = static_cast<const char*>(wpack1_t);
      a.out = part == 0 ? grad_x_src : (part == 1 ? grad_x_dst : grad_x_msg);
      a.part = partials; a.E = num_edges; a.C_k = c_hidden; a.C_n = parts * c_x;
      a.cb0 = part * (c_x / CB); a.n_cb = c_x / CB;
      a.ow = c_x;   // each part's gradient is its own [*, d, c_x] array
      a.ntiles = (num_edges + tile_edges(lmax, mmax, 1, BWD_DX) - 1) / tile_edges(lmax, mmax, 1, BWD_DX);
      a.frags_per_cb = frags_per_cb(lmax, mmax, 1, c_hidden, kc);
      rc = dispatch(lmax, mmax, dtype, 1, BWD_DX, a, s);
      if (rc) return rc;
      // per-edge rows of the message part: single-edge segments, never cut
      if (part == 2) continue;
      rc = fixup(part ? seg_ptr : seg_ptr_src, num_nodes, partials, part ? grad_x_dst : grad_x_src,
                 d * c_x, tile_edges(lmax, mmax, 1, BWD_DX), s);
      if (rc) return rc;
    }
    return MALOQ_OK;
  }
  rc = fixup(seg_ptr_src, num_nodes, partials, grad_x_src, d * c_x, tile_edges(lmax, mmax, 1, BWD_DX), s);
  if (rc) return rc;
  return fixup(seg_ptr, num_nodes, partials, grad_x_dst, d * c_x, tile_edges(lmax, mmax, 1, BWD_DX), s);
}

extern "C" int maloq_message_bwd_dx(int dtype, int lmax, int mmax, int gate, const float* grad_out,
                                    int c_out, const int32_t* dst_by_src,
                                    const int32_t* src_sorted, const int32_t* edge_idx,
                                    int64_t num_edges, const float* dk, const void* rad,
                                    void* grad_rad, const void* r_saved, const void* wpack_t,
                                    const float* jd, float* grad_x, int64_t num_nodes, int c_in,
                                    const int64_t* seg_ptr_src, float* partials, void* dz_ws,
                                    const void* gate_saved, const int32_t* dst_sorted, void* stream) {
  // kernel input channels = c_out (gradient side), output channels = c_in
  int rc = check_common(dtype, lmax, mmax, c_out, c_in, num_edges);
  if (rc) return rc;
  MALOQ_REQUIRE(grad_x && seg_ptr_src && jd && wpack_t, "null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t d = static_cast<int64_t>(lmax + 1) * (lmax + 1);
  if (num_edges > 0) {
    MALOQ_REQUIRE(grad_out && dst_by_src && src_sorted && edge_idx && dk && partials && dz_ws,
                  "null pointer");
    MALOQ_REQUIRE(rad == nullptr || r_saved != nullptr, "the radial gradient needs the saved rows");
    MALOQ_REQUIRE(!gate || gate_saved != nullptr, "the gated backward needs the saved pre-activations");
    PrepArgs p{};
    // rows by edge id either way; in dst-sorted order the gathers of one node's
    // grad_out rows are consecutive
    p.x = grad_out; p.gidx = dst_sorted ? dst_sorted : dst_by_src; p.eidx = dst_sorted ? nullptr : edge_idx;
    p.eulers = nullptr; p.rad = nullptr;
    p.jd = jd; p.y = dz_ws; p.r = nullptr; p.dk = const_cast<float*>(dk); p.build_d = 0;
    p.E = num_edges; p.C = c_out; p.gsave = gate ? gate_saved : nullptr;
    rc = prep_dispatch(lmax, mmax, dtype, BWD_DX, p, s);
    if (rc) return rc;
    Args a{};
    a.a_src = dz_ws; a.dk = dk; a.seg = src_sorted; a.eidx = edge_idx;
    a.rad = rad; a.drad = grad_rad; a.rsave = r_saved;
    a.wpack = static_cast<const char*>(wpack_t); a.bias = nullptr; a.out = grad_x;
    a.part = partials; a.E = num_edges; a.C_k = c_out; a.C_n = c_in; a.n_cb = c_in / CB;
    a.extra = 0; a.ntiles = (num_edges + tile_edges(lmax, mmax, gate, BWD_DX) - 1) / tile_edges(lmax, mmax, gate, BWD_DX);
    const int kc = dtype == 1 ? BF16::KC : F32::KC;
    a.frags_per_cb = frags_per_cb(lmax, mmax, gate, c_out, kc);
    rc = dispatch(lmax, mmax, dtype, gate, BWD_DX, a, s);
    if (rc) return rc;
  }
  return fixup(seg_ptr_src, num_nodes, partials, grad_x, d * c_in, tile_edges(lmax, mmax, gate, BWD_DX), s);
}
