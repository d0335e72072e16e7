// The PyTorch operator layer of the HIP path: the maloq_hip::* operators,
// registered with PyTorch's dispatcher from C++.  Each one checks its
// arguments, allocates its outputs with the caching allocator and calls the C
// ABI of libmaloq_hip.so (include/maloq_hip.h) on the current HIP stream of
// the inputs' device; none has a CPU implementation.  Fake (meta)
// implementations and the autograd formulas are registered from Python
// (maloq_amd/ops.py).  Built with g++ against torch's headers into
// maloq_amd/_maloq_torch.so, which links libmaloq_hip.so.
//
// Operators and the reference interfaces they stand in for:
//   edge_euler(edge_vec, seed)                   wigner_fused.py:403-486 (angles)
//   wigner_from_euler(eulers, lmax, inverse)     rotation.py:189-225 eulers_to_wigner
//   rotate(x, eulers, gather?, lmax, inverse)    bmm(wigner, x[src]), esen_block.py:181,191
//   segment_sum(msg, perm, seg_ptr, n)           index_add_, esen_block.py:205
//   label_transform(x, ...)                      get_net_out / get_H, utils_tensor_decomp.py:154-169
//   message_block_fwd(x, rad?, w0, b0?, wm, ...) Edgewise.forward_node with one SO(2)
//                                                convolution, esen_block.py:146-208
// Private helpers (CPU): _jd_table(), _pack_index(...) expose the tables the
// operators build, for tests.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/maloq_hip.h"
#include "jd_table.h"

namespace {

constexpr int kCB = 32;  // output channels per workgroup of the SO(2) GEMM (fragment column block)

void* stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_rc(int rc, const char* name) {
  TORCH_CHECK(rc == 0, name, " failed (", rc, "): ", maloq_last_error());
}

void require_gpu(const at::Tensor& t, const char* what) {
  TORCH_CHECK_VALUE(t.is_cuda(), "maloq_amd HIP ops need tensors on a ROCm GPU device (", what, ")");
}

int dtype_code(at::ScalarType s) {
  if (s == at::kFloat) return 0;
  if (s == at::kBFloat16) return 1;
  TORCH_CHECK_VALUE(false, "unsupported dtype ", s, " (float32 or bfloat16)");
  return -1;
}

template <class T>
const T* cptr(const c10::optional<at::Tensor>& t) {
  return t.has_value() ? static_cast<const T*>(t->data_ptr()) : nullptr;
}

// Packed J_0 .. J_8 on the device (the table of every lmax <= 8 is its prefix),
// uploaded once per device and kept for the life of the process (never freed:
// the caching allocator may be gone when static destructors run).
const float* jd_on(const at::Device& dev) {
  static std::mutex mu;
  static auto* cache = new std::map<int, at::Tensor>();
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache->find(dev.index());
  if (it == cache->end()) {
    at::Tensor host = at::from_blob(const_cast<float*>(maloq::kJdTable), {maloq::kJdFloats}, at::kFloat);
    it = cache->emplace(dev.index(), host.to(dev)).first;
  }
  return it->second.data_ptr<float>();
}

// ------------------------------------------------------------ weight packing
// Gather index, per packed element, into cat(W0.flatten(), W1.flatten(), ...)
// (fc_m0.weight, then so2_m_conv[m-1].fc.weight).  mode 0: forward GEMM
// (kernel input = c_in side), 1: the input gradient's transposed GEMM.
// Order: output-channel block, kernel-input degree, K step, B fragment of the
// step (per kernel-output degree: g0, [gate], then Wr, Wi for m = 1 ..
// min(mmax, l_k, l_n)), element in the MFMA B operand's lane order.
std::vector<int64_t> pack_index(int code, int lmax, int mmax, bool gate, int c_in, int c_out, int mode,
                                int64_t* total) {
  const bool bf16 = code == 1;
  const int kc = bf16 ? 16 : 8, fe = bf16 ? 512 : 256;
  const int64_t extra = gate ? static_cast<int64_t>(lmax) * c_out : 0;
  const int64_t k0 = static_cast<int64_t>(lmax + 1) * c_in;
  std::vector<int64_t> offs{0, (extra + static_cast<int64_t>(lmax + 1) * c_out) * k0};
  for (int m = 1; m <= mmax; ++m)
    offs.push_back(offs.back() + 2LL * (lmax - m + 1) * c_out * (lmax - m + 1) * c_in);
  *total = offs.back();
  const int c_k = mode == 0 ? c_in : c_out, c_n = mode == 0 ? c_out : c_in;
  const bool gate_out = gate && mode == 0, gate_in = gate && mode == 1;
  std::vector<int64_t> idx;
  for (int cb = 0; cb < c_n / kCB; ++cb)
    for (int l_k = 0; l_k <= lmax; ++l_k) {
      // (kind, m, l_n): kind 0 g0, 1 gate, 2 wr, 3 wi
      std::vector<std::tuple<int, int, int>> frags;
      for (int l_n = 0; l_n <= lmax; ++l_n) {
        frags.emplace_back(0, 0, l_n);
        if ((gate_out && l_n >= 1) || (gate_in && l_k >= 1)) frags.emplace_back(1, 0, l_n);
        const int mm = std::min(mmax, std::min(l_k, l_n));
        for (int m = 1; m <= mm; ++m) {
          frags.emplace_back(2, m, l_n);
          frags.emplace_back(3, m, l_n);
        }
      }
      for (int ks = 0; ks < c_k / kc; ++ks)
        for (const auto& f : frags) {
          const int kind = std::get<0>(f), m = std::get<1>(f), l_n = std::get<2>(f);
          for (int e = 0; e < fe; ++e) {
            const int k_of = bf16 ? (e / 256) * 8 + e % 8 : (e / 128) * 4 + e % 4;
            const int col_of = bf16 ? (e / 8) % 32 : (e / 4) % 32;
            const int64_t cn = static_cast<int64_t>(cb) * kCB + col_of, ck = static_cast<int64_t>(ks) * kc + k_of;
            int64_t c, co;
            int l_in, l_out;
            if (mode == 0) {
              c = ck; co = cn; l_in = l_k; l_out = l_n;
            } else {
              c = cn; co = ck; l_in = l_n; l_out = l_k;
            }
            int64_t v;
            if (kind == 0) {
              v = offs[0] + (extra + static_cast<int64_t>(l_out) * c_out + co) * k0 + static_cast<int64_t>(l_in) * c_in + c;
            } else if (kind == 1) {
              v = offs[0] + (static_cast<int64_t>(l_out - 1) * c_out + co) * k0 + static_cast<int64_t>(l_in) * c_in + c;
            } else {
              const int64_t km = static_cast<int64_t>(lmax - m + 1) * c_in;
              int64_t row = static_cast<int64_t>(l_out - m) * c_out + co;
              if (kind == 3) row += static_cast<int64_t>(lmax - m + 1) * c_out;
              v = offs[m] + row * km + static_cast<int64_t>(l_in - m) * c_in + c;
            }
            idx.push_back(v);
          }
        }
    }
  return idx;
}

// The index on the device, per (dtype, shape, mode, device), built once; every
// entry is checked on the host against the weights' total size.
const at::Tensor& pack_index_on(int code, int lmax, int mmax, bool gate, int c_in, int c_out, int mode,
                                const at::Device& dev, int64_t* total) {
  using Key = std::tuple<int, int, int, bool, int, int, int, int>;
  static std::mutex mu;
  static auto* cache = new std::map<Key, std::pair<at::Tensor, int64_t>>();
  std::lock_guard<std::mutex> lock(mu);
  const Key key{code, lmax, mmax, gate, c_in, c_out, mode, static_cast<int>(dev.index())};
  auto it = cache->find(key);
  if (it == cache->end()) {
    int64_t tot = 0;
    std::vector<int64_t> idx = pack_index(code, lmax, mmax, gate, c_in, c_out, mode, &tot);
    for (int64_t v : idx) TORCH_CHECK(v >= 0 && v < tot, "weight packing index out of range");
    at::Tensor host = at::from_blob(idx.data(), {static_cast<int64_t>(idx.size())}, at::kLong).clone();
    it = cache->emplace(key, std::make_pair(host.to(dev), tot)).first;
  }
  *total = it->second.second;
  return it->second.first;
}

// ------------------------------------------------------------------ Wigner
at::Tensor edge_euler(const at::Tensor& edge_vec, int64_t seed) {
  TORCH_CHECK_VALUE(edge_vec.dim() == 2 && edge_vec.size(1) == 3, "edge_distance_vec must be [E, 3], got ",
                    edge_vec.sizes());
  TORCH_CHECK_VALUE(edge_vec.scalar_type() == at::kFloat, "the HIP Wigner backend computes in fp32; got ",
                    edge_vec.scalar_type());
  require_gpu(edge_vec, "edge_vec");
  const c10::DeviceGuard guard(edge_vec.device());
  const int64_t E = edge_vec.size(0);
  at::Tensor eulers = at::empty({E, 3}, edge_vec.options().dtype(at::kFloat));
  if (E > 0) {
    const at::Tensor v = edge_vec.contiguous();
    check_rc(maloq_edge_euler(v.data_ptr<float>(), E, static_cast<uint64_t>(seed), eulers.data_ptr<float>(),
                              stream_of(v)),
             "maloq_edge_euler");
  }
  return eulers;
}

at::Tensor wigner_from_euler(const at::Tensor& eulers, int64_t lmax, bool inverse) {
  TORCH_CHECK_VALUE(lmax >= 0 && lmax <= 8, "lmax must be 0-8, got ", lmax);
  require_gpu(eulers, "eulers");
  TORCH_CHECK_VALUE(eulers.scalar_type() == at::kFloat && eulers.dim() == 2 && eulers.size(1) == 3,
                    "eulers must be float32 [E, 3]");
  const c10::DeviceGuard guard(eulers.device());
  const int64_t E = eulers.size(0), d = (lmax + 1) * (lmax + 1);
  at::Tensor w = at::empty({E, d, d}, eulers.options());
  if (E > 0) {
    const at::Tensor e = eulers.contiguous();
    float* wp = w.data_ptr<float>();
    check_rc(maloq_wigner_from_euler(e.data_ptr<float>(), E, static_cast<int>(lmax), jd_on(e.device()),
                                     inverse ? nullptr : wp, inverse ? wp : nullptr, 1, stream_of(e)),
             "maloq_wigner_from_euler");
  }
  return w;
}

// ---------------------------------------------------------------- rotation
at::Tensor rotate(const at::Tensor& x, const at::Tensor& eulers, const c10::optional<at::Tensor>& gather,
                  int64_t lmax, bool inverse) {
  const int code = dtype_code(x.scalar_type());
  TORCH_CHECK_VALUE(lmax >= 0 && lmax <= 8, "lmax must be 0-8, got ", lmax);
  const int64_t d = (lmax + 1) * (lmax + 1);
  TORCH_CHECK_VALUE(x.dim() == 3 && x.size(1) == d, "x must be [*, ", d, ", C], got ", x.sizes());
  const int64_t C = x.size(2);
  TORCH_CHECK_VALUE(C % 4 == 0, "channels must be a multiple of 4");
  require_gpu(x, "x");
  require_gpu(eulers, "eulers");
  if (gather.has_value()) require_gpu(*gather, "gather");
  const c10::DeviceGuard guard(x.device());
  const int64_t E = eulers.size(0);
  TORCH_CHECK_VALUE(eulers.dim() == 2 && eulers.size(1) == 3, "eulers must be [E, 3]");
  const at::Tensor eul = eulers.to(at::kFloat).contiguous();
  at::Tensor g;
  if (gather.has_value()) {
    TORCH_CHECK_VALUE(gather->dim() == 1 && gather->size(0) == E, "gather must be [E]");
    if (E > 0) {
      // the kernel gathers without bounds checks (one host sync, as on the reference's indexing path)
      const int64_t lo = gather->min().item<int64_t>(), hi = gather->max().item<int64_t>();
      TORCH_CHECK_VALUE(lo >= 0 && hi < x.size(0), "gather holds rows outside x");
    }
    g = gather->to(at::kInt).contiguous();
  } else {
    TORCH_CHECK_VALUE(x.size(0) == E, "without gather, x must have one row per edge");
  }
  at::Tensor out = at::empty({E, d, C}, x.options());
  if (E == 0) return out;
  const at::Tensor xc = x.contiguous();
  check_rc(maloq_rotate(code, code, static_cast<int>(lmax), xc.data_ptr(), static_cast<int>(C),
                        g.defined() ? g.data_ptr<int32_t>() : nullptr, E, eul.data_ptr<float>(), nullptr,
                        jd_on(x.device()), inverse ? 1 : 0, out.data_ptr(), stream_of(xc)),
           "maloq_rotate");
  return out;
}

// ------------------------------------------------------------- segment sum
at::Tensor segment_sum(const at::Tensor& msg, const at::Tensor& perm, const at::Tensor& seg_ptr,
                       int64_t num_segments) {
  require_gpu(msg, "msg");
  require_gpu(perm, "perm");
  require_gpu(seg_ptr, "seg_ptr");
  TORCH_CHECK_VALUE(msg.dim() >= 1 && num_segments >= 0, "msg must have a leading edge dimension");
  const c10::DeviceGuard guard(msg.device());
  const at::Tensor m = msg.to(at::kFloat).contiguous();
  std::vector<int64_t> shape{num_segments};
  int64_t width = 1;
  for (int64_t k = 1; k < msg.dim(); ++k) {
    shape.push_back(msg.size(k));
    width *= msg.size(k);
  }
  at::Tensor out = at::empty(shape, msg.options().dtype(at::kFloat));
  const at::Tensor p = perm.to(at::kLong).contiguous(), s = seg_ptr.to(at::kLong).contiguous();
  check_rc(maloq_segment_sum(m.data_ptr<float>(), p.data_ptr<int64_t>(), s.data_ptr<int64_t>(), num_segments,
                             width, out.data_ptr<float>(), stream_of(m)),
           "maloq_segment_sum");
  return out;
}

// --------------------------------------------------------- basis transform
// Rows of several column groups (ngroups > 1) are permuted by a separate
// column gather: the input through perm_inv (the inverse of perm_in), the
// output through perm_out.
at::Tensor label_transform(const at::Tensor& x, const at::Tensor& blocks, const c10::optional<at::Tensor>& w,
                           const at::Tensor& sched, const c10::optional<at::Tensor>& perm_in,
                           const c10::optional<at::Tensor>& perm_out, int64_t num_blocks, int64_t ngroups,
                           int64_t group_cols, const c10::optional<at::Tensor>& perm_inv) {
  require_gpu(x, "x");
  TORCH_CHECK_VALUE(x.dim() == 2, "label rows must be [R, t]");
  TORCH_CHECK_VALUE(x.scalar_type() == at::kFloat, "label rows must be float32");
  const c10::DeviceGuard guard(x.device());
  at::Tensor xc = x.contiguous();
  const bool pre = ngroups > 1 && perm_in.has_value();
  const bool post = ngroups > 1 && perm_out.has_value();
  at::Tensor ones;
  if (pre || post) ones = at::ones({xc.size(1)}, xc.options());
  auto gather = [&](const at::Tensor& y, const at::Tensor& src) {
    at::Tensor o = at::empty_like(y);
    check_rc(maloq_gather_columns(y.data_ptr<float>(), y.size(1), y.size(0), src.data_ptr<int32_t>(),
                                  ones.data_ptr<float>(), static_cast<int>(y.size(1)), o.data_ptr<float>(),
                                  o.size(1), stream_of(y)),
             "maloq_gather_columns");
    return o;
  };
  if (pre) {
    TORCH_CHECK_VALUE(perm_inv.has_value(), "rows of several column groups need the inverse input permutation");
    xc = gather(xc, *perm_inv);
  }
  at::Tensor out = at::empty_like(xc);
  check_rc(maloq_label_transform(xc.data_ptr<float>(), pre ? nullptr : cptr<int32_t>(perm_in),
                                 out.data_ptr<float>(), post ? nullptr : cptr<int32_t>(perm_out), xc.size(0),
                                 static_cast<int>(xc.size(1)), static_cast<int>(num_blocks),
                                 blocks.data_ptr<int32_t>(), cptr<float>(w), sched.data_ptr<int32_t>(),
                                 static_cast<int>(ngroups), static_cast<int>(group_cols), stream_of(xc)),
           "maloq_label_transform");
  return post ? gather(out, *perm_out) : out;
}

// ----------------------------------------------------------- message block
// Node output and the workspaces the backward reads: [out, y, r, dk, g]
// (r empty without radial scales, g empty ungated); src, dst, seg_ptr and
// eulers are those of the dst-sorted graph plan.
std::vector<at::Tensor> message_block_fwd(const at::Tensor& x, const c10::optional<at::Tensor>& rad,
                                          const at::Tensor& w0, const c10::optional<at::Tensor>& b0,
                                          at::TensorList wm, const at::Tensor& src, const at::Tensor& dst,
                                          const at::Tensor& seg_ptr, const at::Tensor& eulers, int64_t lmax,
                                          int64_t mmax, bool gate) {
  const int code = dtype_code(x.scalar_type());
  require_gpu(x, "x");
  require_gpu(eulers, "eulers");
  require_gpu(w0, "w0");
  TORCH_CHECK_VALUE(maloq_message_supported(static_cast<int>(lmax), static_cast<int>(mmax)),
                    "no message kernels for lmax=", lmax, ", mmax=", mmax);
  const int64_t d = (lmax + 1) * (lmax + 1);
  TORCH_CHECK_VALUE(x.dim() == 3 && x.size(1) == d, "x must be [N, (lmax+1)^2, C]");
  TORCH_CHECK_VALUE(src.scalar_type() == at::kInt && dst.scalar_type() == at::kInt &&
                        seg_ptr.scalar_type() == at::kLong,
                    "the plan's src/dst must be int32 and seg_ptr int64");
  TORCH_CHECK_VALUE(static_cast<int64_t>(wm.size()) >= mmax, "wm needs mmax weights");
  const c10::DeviceGuard guard(x.device());
  const int64_t c_in = x.size(2), n0 = w0.size(0);
  const int64_t c_out = n0 / (lmax + 1 + (gate ? lmax : 0));
  const int64_t E = src.size(0), num_nodes = seg_ptr.size(0) - 1;
  const int kr = maloq_message_kept_rows(static_cast<int>(lmax), static_cast<int>(mmax));
  const auto dt = x.scalar_type();
  const at::Device dev = x.device();
  // weights in fragment order
  int64_t total = 0;
  const at::Tensor& idx = pack_index_on(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                        static_cast<int>(c_in), static_cast<int>(c_out), 0, dev, &total);
  std::vector<at::Tensor> srcs{w0.detach().to(at::kFloat).contiguous()};
  for (int64_t m = 0; m < mmax; ++m) srcs.push_back(wm[m].detach().to(at::kFloat).contiguous());
  int64_t have = 0;
  std::vector<const float*> sp;
  std::vector<int64_t> sn;
  for (const auto& t : srcs) {
    have += t.numel();
    sp.push_back(t.data_ptr<float>());
    sn.push_back(t.numel());
  }
  TORCH_CHECK_VALUE(have == total, "weight shapes do not match (lmax, mmax, channels)");
  const int64_t want = maloq_message_wpack_bytes(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                                 static_cast<int>(c_in), static_cast<int>(c_out));
  at::Tensor wpack = at::empty({idx.numel()}, x.options().dtype(dt));
  TORCH_CHECK(wpack.numel() * wpack.element_size() == want, "packed weight size mismatch");
  check_rc(maloq_message_pack(code, static_cast<int>(sp.size()), sp.data(), sn.data(), idx.data_ptr<int64_t>(),
                              idx.numel(), wpack.data_ptr(), stream_of(x)),
           "maloq_message_pack");
  // outputs and workspaces
  at::Tensor out = at::empty({num_nodes, d, c_out}, x.options().dtype(at::kFloat));
  const int64_t pf = maloq_message_partials_floats(static_cast<int>(lmax), gate ? 1 : 0, E, static_cast<int>(c_out));
  at::Tensor parts = at::empty({pf > 1 ? pf : 1}, x.options().dtype(at::kFloat));
  at::Tensor radc;
  if (rad.has_value()) {
    int64_t rw = 0;
    for (int64_t m = 0; m <= mmax; ++m) rw += (lmax - m + 1) * c_in;
    TORCH_CHECK_VALUE(rad->dim() == 2 && rad->size(0) == E && rad->size(1) == rw,
                      "rad must be [E, sum_m (lmax-m+1) C_in]");
    radc = rad->to(dt).contiguous();
  }
  // saved rows: rows past E are zero (the bf16 weight gradient reads whole chunks)
  const int64_t rows = maloq_message_edge_rows(E);
  at::Tensor y = at::empty({rows, kr, c_in}, x.options());
  if (rows > E) y.narrow(0, E, rows - E).zero_();
  const int64_t E1 = E > 1 ? E : 1;
  at::Tensor r = rad.has_value() ? at::empty({E1, kr, c_in}, x.options()) : at::empty({0}, x.options());
  TORCH_CHECK_VALUE(eulers.dim() == 2 && eulers.size(0) == E && eulers.size(1) == 3,
                    "eulers must be [E, 3] (dst-sorted)");
  const at::Tensor eul = eulers.to(at::kFloat).contiguous();
  at::Tensor dk = at::empty({E1, maloq_message_wigner_floats(static_cast<int>(lmax), static_cast<int>(mmax))},
                            x.options().dtype(at::kFloat));
  at::Tensor g = gate ? at::empty({E1, kr + lmax, c_out}, x.options()) : at::empty({0}, x.options());
  at::Tensor bias;
  if (b0.has_value()) bias = b0->to(at::kFloat).contiguous();
  const at::Tensor xc = x.contiguous();
  check_rc(maloq_message_fwd(code, static_cast<int>(lmax), static_cast<int>(mmax), gate ? 1 : 0, xc.data_ptr(),
                             static_cast<int>(c_in), src.data_ptr<int32_t>(), dst.data_ptr<int32_t>(), E,
                             eul.data_ptr<float>(), radc.defined() ? radc.data_ptr() : nullptr, wpack.data_ptr(),
                             bias.defined() ? bias.data_ptr<float>() : nullptr, jd_on(dev), out.data_ptr<float>(),
                             num_nodes, static_cast<int>(c_out), seg_ptr.data_ptr<int64_t>(),
                             parts.data_ptr<float>(), y.data_ptr(), rad.has_value() ? r.data_ptr() : nullptr,
                             dk.data_ptr<float>(), gate ? g.data_ptr() : nullptr, stream_of(xc)),
           "maloq_message_fwd");
  return {out, y, r, dk, g};
}

// ------------------------------------------------------- test-only helpers
at::Tensor jd_table() {
  return at::from_blob(const_cast<float*>(maloq::kJdTable), {maloq::kJdFloats}, at::kFloat).clone();
}

at::Tensor pack_index_cpu(int64_t code, int64_t lmax, int64_t mmax, bool gate, int64_t c_in, int64_t c_out,
                          int64_t mode) {
  int64_t total = 0;
  std::vector<int64_t> idx = pack_index(static_cast<int>(code), static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                        static_cast<int>(c_in), static_cast<int>(c_out), static_cast<int>(mode),
                                        &total);
  return at::from_blob(idx.data(), {static_cast<int64_t>(idx.size())}, at::kLong).clone();
}

}  // namespace

TORCH_LIBRARY(maloq_hip, m) {
  m.def("edge_euler(Tensor edge_vec, int seed) -> Tensor");
  m.def("wigner_from_euler(Tensor eulers, int lmax, bool inverse) -> Tensor");
  m.def("rotate(Tensor x, Tensor eulers, Tensor? gather, int lmax, bool inverse) -> Tensor");
  m.def("segment_sum(Tensor msg, Tensor perm, Tensor seg_ptr, int num_segments) -> Tensor");
  m.def("label_transform(Tensor x, Tensor blocks, Tensor? w, Tensor sched, Tensor? perm_in, Tensor? perm_out, "
        "int num_blocks, int ngroups, int group_cols, Tensor? perm_inv) -> Tensor");
  m.def("message_block_fwd(Tensor x, Tensor? rad, Tensor w0, Tensor? b0, Tensor[] wm, Tensor src, Tensor dst, "
        "Tensor seg_ptr, Tensor eulers, int lmax, int mmax, bool gate) -> Tensor[]");
  m.def("_jd_table() -> Tensor", &jd_table);
  m.def("_pack_index(int dtype_code, int lmax, int mmax, bool gate, int c_in, int c_out, int mode) -> Tensor",
        &pack_index_cpu);
}

TORCH_LIBRARY_IMPL(maloq_hip, CUDA, m) {
  m.impl("edge_euler", &edge_euler);
  m.impl("wigner_from_euler", &wigner_from_euler);
  m.impl("rotate", &rotate);
  m.impl("segment_sum", &segment_sum);
  m.impl("label_transform", &label_transform);
  m.impl("message_block_fwd", &message_block_fwd);
}
