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
//   edge_vec_to_wigner(edge_vec, jd, lmax, seed, ..)  edge_vec_to_wigner_fused, wigner_fused.py:403-486,
//                                                and the (wigner, wigner_inv) pair, esen_osh.py:266-296
//   wigner_from_euler(eulers, lmax, inverse)     rotation.py:189-225 eulers_to_wigner
//   rotate(x, eulers, gather?, lmax, inverse)    bmm(wigner, x[src]), esen_block.py:181,191
//   segment_sum(msg, perm, seg_ptr, n)           index_add_, esen_block.py:205
//   label_transform(x, ...)                      get_net_out / get_H, utils_tensor_decomp.py:154-169
//   message_block_fwd(x, rad?, w0, b0?, wm, ...) Edgewise.forward_node with one SO(2)
//                                                convolution, esen_block.py:146-208
//   message_block_bwd(grad_out, ...)             its autograd backward (so2_layers.py:139-214)
//   basis_row_meta(...)                          the row plan of the fused Fock transforms
//   fock_to_irreps(fock, ...)                    matrix2label + get_net_out,
//                                                fock_targets_batched.py:335-464
//   irreps_to_fock(net_out, fock!, ...)          get_H + label2matrix (in place),
//                                                splittrainer.py:1172-1233
// Private helpers (CPU): _jd_table(), _pack_index(...) expose the tables the
// operators build, for tests.
#include <ATen/ATen.h>
#include <ATen/hip/HIPContextLight.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <cstdint>
#include <initializer_list>
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

// Device pointer of an optional tensor of element type T (null if absent);
// a tensor of another dtype is refused rather than reinterpreted.
template <class T>
const T* cptr(const c10::optional<at::Tensor>& t) {
  return t.has_value() ? t->data_ptr<T>() : nullptr;
}

// Every given tensor on the device of `ref` (the kernels take raw pointers).
void same_device(const at::Tensor& ref, std::initializer_list<c10::optional<at::Tensor>> ts) {
  for (const auto& t : ts)
    TORCH_CHECK_VALUE(!t.has_value() || t->device() == ref.device(), "all tensors must be on ", ref.device(),
                      ", got one on ", t->device());
}

// 1-D length of an index tensor (or -1 if absent).
int64_t len(const c10::optional<at::Tensor>& t) { return t.has_value() ? t->numel() : -1; }

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

// Dense block-diagonal Wigner-D [E, d, d] from edge vectors in one launch,
// with the packed J_0..J_lmax given by the caller (its Jd): [D] or, with
// with_inverse, [D, D^T]; with_eulers appends the Euler triples used [E, 3].
std::vector<at::Tensor> edge_vec_to_wigner(const at::Tensor& edge_vec, const at::Tensor& jd, int64_t lmax,
                                           int64_t seed, bool with_inverse, bool with_eulers) {
  TORCH_CHECK_VALUE(lmax >= 0 && lmax <= 8, "lmax must be 0-8, got ", lmax);
  TORCH_CHECK_VALUE(edge_vec.dim() == 2 && edge_vec.size(1) == 3, "edge_distance_vec must be [E, 3], got ",
                    edge_vec.sizes());
  TORCH_CHECK_VALUE(edge_vec.scalar_type() == at::kFloat, "the HIP Wigner backend computes in fp32; got ",
                    edge_vec.scalar_type());
  require_gpu(edge_vec, "edge_vec");
  int64_t need = 0;
  for (int64_t l = 0; l <= lmax; ++l) need += (2 * l + 1) * (2 * l + 1);
  TORCH_CHECK_VALUE(jd.scalar_type() == at::kFloat && jd.is_contiguous() && jd.numel() >= need,
                    "jd must hold the packed fp32 J_0..J_lmax (", need, " floats)");
  same_device(edge_vec, {jd});
  const c10::DeviceGuard guard(edge_vec.device());
  const int64_t E = edge_vec.size(0), d = (lmax + 1) * (lmax + 1);
  std::vector<at::Tensor> res{at::empty({E, d, d}, edge_vec.options())};
  if (with_inverse) res.push_back(at::empty({E, d, d}, edge_vec.options()));
  if (with_eulers) res.push_back(at::empty({E, 3}, edge_vec.options()));
  if (E == 0) return res;
  const at::Tensor v = edge_vec.contiguous();
  check_rc(maloq_edge_vec_to_wigner(v.data_ptr<float>(), E, static_cast<uint64_t>(seed), static_cast<int>(lmax),
                                    jd.data_ptr<float>(), with_eulers ? res.back().data_ptr<float>() : nullptr,
                                    res[0].data_ptr<float>(), with_inverse ? res[1].data_ptr<float>() : nullptr, 1,
                                    stream_of(v)),
           "maloq_edge_vec_to_wigner");
  return res;
}

// The same into a caller's out [E, d, d] (contiguous fp32): only the diagonal
// blocks are written, as the reference's out= contract states.
void edge_vec_to_wigner_out(const at::Tensor& edge_vec, const at::Tensor& jd, int64_t lmax, int64_t seed,
                            const at::Tensor& out) {
  TORCH_CHECK_VALUE(lmax >= 0 && lmax <= 8, "lmax must be 0-8, got ", lmax);
  TORCH_CHECK_VALUE(edge_vec.dim() == 2 && edge_vec.size(1) == 3 && edge_vec.scalar_type() == at::kFloat,
                    "edge_distance_vec must be float32 [E, 3]");
  require_gpu(edge_vec, "edge_vec");
  const int64_t E = edge_vec.size(0), d = (lmax + 1) * (lmax + 1);
  TORCH_CHECK_VALUE(out.dim() == 3 && out.size(0) == E && out.size(1) == d && out.size(2) == d &&
                        out.is_contiguous() && out.scalar_type() == at::kFloat,
                    "out must be contiguous float32 [E, d, d]");
  int64_t need = 0;
  for (int64_t l = 0; l <= lmax; ++l) need += (2 * l + 1) * (2 * l + 1);
  TORCH_CHECK_VALUE(jd.scalar_type() == at::kFloat && jd.is_contiguous() && jd.numel() >= need,
                    "jd must hold the packed fp32 J_0..J_lmax (", need, " floats)");
  same_device(edge_vec, {jd, out});
  const c10::DeviceGuard guard(edge_vec.device());
  if (E == 0) return;
  const at::Tensor v = edge_vec.contiguous();
  check_rc(maloq_edge_vec_to_wigner(v.data_ptr<float>(), E, static_cast<uint64_t>(seed), static_cast<int>(lmax),
                                    jd.data_ptr<float>(), nullptr, out.data_ptr<float>(), nullptr, 0, stream_of(v)),
           "maloq_edge_vec_to_wigner");
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
  same_device(x, {eulers, gather});
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
  TORCH_CHECK_VALUE(perm.numel() == msg.size(0), "perm must hold one entry per message row");
  TORCH_CHECK_VALUE(seg_ptr.numel() == num_segments + 1, "seg_ptr must hold num_segments + 1 offsets");
  same_device(msg, {perm, seg_ptr});
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
  same_device(x, {blocks, w, sched, perm_in, perm_out, perm_inv});
  TORCH_CHECK_VALUE(blocks.numel() == 4 * num_blocks, "blocks must be [num_blocks, 4]");
  for (const auto* p : {&perm_in, &perm_out, &perm_inv})
    TORCH_CHECK_VALUE(len(*p) < 0 || len(*p) == x.size(1), "column permutations must have one entry per column");
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
  TORCH_CHECK_VALUE(dst.numel() == src.numel() && seg_ptr.numel() >= 1, "src and dst must have one entry per edge");
  same_device(x, {rad, w0, b0, src, dst, seg_ptr, eulers});
  for (int64_t m = 0; m < mmax; ++m) same_device(x, {wm[m]});
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

// Saved rows of the bf16 weight gradient: rows past E are zero (it reads whole
// 128-edge chunks).
at::Tensor edge_rows(int64_t E, int64_t rows, int64_t c, const at::TensorOptions& opt) {
  const int64_t n = maloq_message_edge_rows(E);
  at::Tensor t = at::empty({n, rows, c}, opt);
  if (n > E) t.narrow(0, E, n - E).zero_();
  return t;
}

at::Tensor pack_weights(int code, int64_t lmax, int64_t mmax, bool gate, int64_t c_in, int64_t c_out, int mode,
                        const at::Tensor& w0, at::TensorList wm, at::ScalarType dt) {
  int64_t total = 0;
  const at::Tensor& idx = pack_index_on(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                        static_cast<int>(c_in), static_cast<int>(c_out), mode, w0.device(), &total);
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
  const int64_t c_k = mode == 0 ? c_in : c_out, c_n = mode == 0 ? c_out : c_in;
  const int64_t want = maloq_message_wpack_bytes(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                                 static_cast<int>(c_k), static_cast<int>(c_n));
  at::Tensor wpack = at::empty({idx.numel()}, w0.options().dtype(dt));
  TORCH_CHECK(wpack.numel() * wpack.element_size() == want, "packed weight size mismatch");
  check_rc(maloq_message_pack(code, static_cast<int>(sp.size()), sp.data(), sn.data(), idx.data_ptr<int64_t>(),
                              idx.numel(), wpack.data_ptr(), stream_of(w0)),
           "maloq_message_pack");
  return wpack;
}

// Split-K count of the weight gradient over the edges (deterministic: the
// partials are summed in split order).  bf16: 256 x 256 output tiles, one
// workgroup per CU, the most splits that keep every workgroup in one round;
// fp32: 128 x 128 tiles, the count that balances the workgroups over the CUs
// (at most three per CU, >= 1024 edges per split).
int dw_splits(bool bf16, int64_t lmax, int64_t mmax, bool gate, int64_t c_out, int64_t c_in, int64_t E, int cus) {
  std::vector<std::pair<int64_t, int64_t>> groups{{lmax + 1, lmax + 1}};
  for (int64_t m = 1; m <= mmax; ++m) groups.emplace_back(2 * (lmax - m + 1), 2 * (lmax - m + 1));
  if (gate) groups.emplace_back(lmax, lmax + 1);
  auto cdiv = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
  int64_t ntiles = 0;
  const int64_t tile = bf16 ? 256 : 128;
  for (const auto& g : groups) ntiles += cdiv(g.first * c_out, tile) * cdiv(g.second * c_in, tile);
  if (bf16) return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({64, cus / ntiles, cdiv(E, 128)})));
  int best = 1;
  double best_cost = 0;
  bool have = false;
  for (int s = 1; s <= 16; ++s) {
    if (ntiles * s > 3 * cus || s > std::max<int64_t>(1, E / 1024)) continue;
    const double cost = static_cast<double>(cdiv(ntiles * s, cus)) / s;
    // ties go to the larger split count
    if (!have || cost < best_cost || (cost == best_cost && s > best)) {
      best = s;
      best_cost = cost;
      have = true;
    }
  }
  return best;
}

// Gradients of message_block_fwd from its saved rows: [grad_x fp32 [N, d, c_in],
// grad_rad (empty unless asked), dW0, db0, dW_1 .. dW_mmax] (fp32).  The
// graph arrives as the plan's source-sorted arrays: bwd_src, bwd_dst,
// bwd_eidx (dst-sorted position of each source-sorted edge), seg_ptr_src.
std::vector<at::Tensor> message_block_bwd(const at::Tensor& grad_out, const c10::optional<at::Tensor>& rad,
                                          const at::Tensor& w0, at::TensorList wm, const at::Tensor& bwd_src,
                                          const at::Tensor& bwd_dst, const at::Tensor& bwd_eidx,
                                          const at::Tensor& seg_ptr_src, const at::Tensor& y, const at::Tensor& dk,
                                          const c10::optional<at::Tensor>& r, const c10::optional<at::Tensor>& g,
                                          int64_t num_nodes, int64_t c_in, int64_t lmax, int64_t mmax, bool gate,
                                          bool need_rad_grad) {
  const auto dt = y.scalar_type();
  const int code = dtype_code(dt);
  require_gpu(grad_out, "grad_out");
  require_gpu(y, "y");
  require_gpu(dk, "dk");
  TORCH_CHECK_VALUE(maloq_message_supported(static_cast<int>(lmax), static_cast<int>(mmax)),
                    "no message kernels for lmax=", lmax, ", mmax=", mmax);
  const int64_t d = (lmax + 1) * (lmax + 1);
  TORCH_CHECK_VALUE(grad_out.dim() == 3 && grad_out.size(1) == d, "grad_out must be [N, (lmax+1)^2, c_out]");
  TORCH_CHECK_VALUE(bwd_src.scalar_type() == at::kInt && bwd_dst.scalar_type() == at::kInt &&
                        bwd_eidx.scalar_type() == at::kInt && seg_ptr_src.scalar_type() == at::kLong,
                    "the plan's source-sorted arrays must be int32 and seg_ptr_src int64");
  TORCH_CHECK_VALUE(static_cast<int64_t>(wm.size()) >= mmax, "wm needs mmax weights");
  TORCH_CHECK_VALUE(!gate || (g.has_value() && g->numel() > 0),
                    "the gated backward needs the forward's pre-activation rows");
  TORCH_CHECK_VALUE(bwd_dst.numel() == bwd_src.numel() && bwd_eidx.numel() == bwd_src.numel(),
                    "the source-sorted arrays must have one entry per edge");
  TORCH_CHECK_VALUE(seg_ptr_src.numel() == num_nodes + 1, "seg_ptr_src must hold num_nodes + 1 offsets");
  TORCH_CHECK_VALUE(y.dim() == 3 && y.size(0) >= bwd_src.numel() && dk.size(0) >= bwd_src.numel(),
                    "the saved rows must cover every edge");
  same_device(grad_out, {rad, w0, bwd_src, bwd_dst, bwd_eidx, seg_ptr_src, y, dk, r, g});
  for (int64_t m = 0; m < mmax; ++m) same_device(grad_out, {wm[m]});
  const c10::DeviceGuard guard(grad_out.device());
  const int64_t c_out = grad_out.size(2), E = bwd_src.size(0);
  const int kr = maloq_message_kept_rows(static_cast<int>(lmax), static_cast<int>(mmax));
  const auto opt32 = grad_out.options().dtype(at::kFloat);
  void* st = stream_of(grad_out);
  // input gradient (and the radial gradient)
  const at::Tensor wpack_t = pack_weights(code, lmax, mmax, gate, c_in, c_out, 1, w0, wm, dt);
  at::Tensor gx = at::empty({num_nodes, d, c_in}, opt32);
  const int64_t pf = maloq_message_partials_floats(static_cast<int>(lmax), gate ? 1 : 0, E, static_cast<int>(c_in));
  at::Tensor parts = at::empty({pf > 1 ? pf : 1}, opt32);
  at::Tensor radc, grad_rad = at::empty({0}, opt32);
  if (rad.has_value()) {
    radc = rad->to(dt).contiguous();
    if (need_rad_grad) grad_rad = at::empty_like(radc);
  }
  at::Tensor dz = edge_rows(E, kr + (gate ? lmax : 0), c_out, y.options());
  const at::Tensor gq = grad_out.to(at::kFloat).contiguous();
  const bool has_r = r.has_value() && r->numel() > 0;
  check_rc(maloq_message_bwd_dx(code, static_cast<int>(lmax), static_cast<int>(mmax), gate ? 1 : 0,
                                gq.data_ptr<float>(), static_cast<int>(c_out), bwd_dst.data_ptr<int32_t>(),
                                bwd_src.data_ptr<int32_t>(), bwd_eidx.data_ptr<int32_t>(), E, dk.data_ptr<float>(),
                                radc.defined() ? radc.data_ptr() : nullptr,
                                grad_rad.numel() ? grad_rad.data_ptr() : nullptr, has_r ? r->data_ptr() : nullptr,
                                wpack_t.data_ptr(), jd_on(grad_out.device()), gx.data_ptr<float>(), num_nodes,
                                static_cast<int>(c_in), seg_ptr_src.data_ptr<int64_t>(), parts.data_ptr<float>(),
                                dz.data_ptr(), gate ? g->data_ptr() : nullptr, st),
           "maloq_message_bwd_dx");
  // weight and bias gradients
  const int64_t extra = gate ? lmax * c_out : 0;
  at::Tensor dw0, db0;
  std::vector<at::Tensor> dwm;
  if (E == 0) {
    dw0 = at::zeros({extra + (lmax + 1) * c_out, (lmax + 1) * c_in}, opt32);
    for (int64_t m = 1; m <= mmax; ++m) dwm.push_back(at::zeros({2 * (lmax - m + 1) * c_out, (lmax - m + 1) * c_in}, opt32));
    db0 = at::zeros({extra + (lmax + 1) * c_out}, opt32);
  } else {
    if (dt == at::kBFloat16)
      TORCH_CHECK(dz.size(0) >= maloq_message_edge_rows(E) && y.size(0) == dz.size(0),
                  "bf16 weight gradient needs the padded workspaces");
    const int cus = at::cuda::getDeviceProperties(grad_out.device().index())->multiProcessorCount;
    const int splits = dw_splits(dt == at::kBFloat16, lmax, mmax, gate, c_out, c_in, E, cus);
    const int64_t dp = maloq_message_dw_partials_floats(static_cast<int>(lmax), static_cast<int>(mmax), gate ? 1 : 0,
                                                        static_cast<int>(c_out), static_cast<int>(c_in), splits);
    at::Tensor dparts = at::empty({dp > 1 ? dp : 1}, opt32);
    dw0 = at::empty({extra + (lmax + 1) * c_out, (lmax + 1) * c_in}, opt32);
    std::vector<float*> dptr;
    for (int64_t m = 1; m <= mmax; ++m) {
      dwm.push_back(at::empty({2 * (lmax - m + 1) * c_out, (lmax - m + 1) * c_in}, opt32));
      dptr.push_back(dwm.back().data_ptr<float>());
    }
    if (dptr.empty()) dptr.push_back(nullptr);
    check_rc(maloq_message_dw(code, static_cast<int>(lmax), static_cast<int>(mmax), gate ? 1 : 0, dz.data_ptr(),
                              y.data_ptr(), E, static_cast<int>(c_out), static_cast<int>(c_in), splits,
                              dparts.data_ptr<float>(), dw0.data_ptr<float>(), dptr.data(), st),
             "maloq_message_dw");
    db0 = at::empty({extra + (lmax + 1) * c_out}, opt32);
    const int rpe = static_cast<int>(dz.size(1));
    // (first row, rows, output offset): the m = 0 rows, then a gated block's gate rows
    std::vector<std::tuple<int, int, int64_t>> groups{{0, static_cast<int>(lmax + 1), extra}};
    if (gate) groups.emplace_back(kr, static_cast<int>(lmax), 0);
    int64_t cs_n = 1;
    for (const auto& gr : groups)
      cs_n = std::max(cs_n, maloq_message_colsum_partials_floats(std::get<1>(gr), static_cast<int>(c_out), E));
    at::Tensor cs = at::empty({cs_n}, opt32);
    for (const auto& gr : groups)
      check_rc(maloq_message_colsum(code, dz.data_ptr(), rpe, std::get<0>(gr), std::get<1>(gr), static_cast<int>(c_out),
                                    E, cs.data_ptr<float>(), db0.data_ptr<float>() + std::get<2>(gr), st),
               "maloq_message_colsum");
  }
  std::vector<at::Tensor> res{gx, grad_rad, dw0, db0};
  for (auto& t : dwm) res.push_back(t);
  return res;
}

// ------------------------------------------------ fused Fock <-> irreps
// The tables (pair_kind, slots, kind_blocks, blocks, w, sched) are those of a
// basis_transform.HipE3TensorDecomp; ld > 0: dense Fock rows of stride ld (the
// tensor's own row stride, unit column stride), ld = 0: block-list storage
// with block_data_offsets.
at::Tensor basis_row_meta(int64_t ld, const c10::optional<at::Tensor>& bdo, const at::Tensor& off,
                          const at::Tensor& Z, const at::Tensor& rows, const at::Tensor& cols,
                          const at::Tensor& pair_kind, int64_t maxe) {
  require_gpu(rows, "rows");
  TORCH_CHECK_VALUE(cols.numel() == rows.numel(), "rows and cols must have the same length");
  TORCH_CHECK_VALUE(len(bdo) < 0 || len(bdo) >= rows.numel(), "block_data_offsets must cover every pair");
  same_device(rows, {bdo, off, Z, cols, pair_kind});
  const c10::DeviceGuard guard(rows.device());
  const int64_t R = rows.size(0);
  at::Tensor meta = at::empty({R > 1 ? R : 1, 4}, rows.options().dtype(at::kInt));
  check_rc(maloq_basis_row_meta(ld, cptr<int64_t>(bdo), off.data_ptr<int32_t>(), Z.data_ptr<int32_t>(),
                                rows.data_ptr<int32_t>(), cols.data_ptr<int32_t>(), R, pair_kind.data_ptr<int32_t>(),
                                static_cast<int>(maxe), meta.data_ptr<int32_t>(), stream_of(rows)),
           "maloq_basis_row_meta");
  return meta;
}

// Shapes a fused Fock call relies on: the row plan (or the pair list) covers
// num_rows rows; the CG block table has num_blocks entries; every tensor on
// the Fock matrix's device.
void check_fock_args(const at::Tensor& fock, const c10::optional<at::Tensor>& bdo,
                     const c10::optional<at::Tensor>& off, const c10::optional<at::Tensor>& Z,
                     const c10::optional<at::Tensor>& rows, const c10::optional<at::Tensor>& cols,
                     const c10::optional<at::Tensor>& meta, int64_t num_rows, int64_t t, const at::Tensor& blocks,
                     int64_t num_blocks, std::initializer_list<c10::optional<at::Tensor>> tables) {
  TORCH_CHECK_VALUE(num_rows >= 0 && t > 0, "bad row count or width");
  TORCH_CHECK_VALUE(blocks.numel() == 4 * num_blocks, "blocks must be [num_blocks, 4]");
  if (meta.has_value()) {
    TORCH_CHECK_VALUE(meta->dim() == 2 && meta->size(1) == 4 && meta->size(0) >= num_rows,
                      "the row plan must hold num_rows [4] entries");
  } else if (rows.has_value() && cols.has_value()) {
    TORCH_CHECK_VALUE(rows->numel() == num_rows && cols->numel() == num_rows,
                      "rows and cols must hold num_rows entries");
    TORCH_CHECK_VALUE(len(bdo) < 0 || len(bdo) >= num_rows, "block_data_offsets must cover every pair");
  }
  same_device(fock, {bdo, off, Z, rows, cols, meta, blocks});
  same_device(fock, tables);
}

// One launch: from the row plan `meta` (num_rows rows) or, without one, from
// the pair list (off, Z, rows, cols, block_data_offsets).  perm_post: rows of
// several column groups are sorted by a separate column gather afterwards.
at::Tensor fock_to_irreps(const at::Tensor& fock, int64_t ld, const c10::optional<at::Tensor>& bdo,
                          const c10::optional<at::Tensor>& off, const c10::optional<at::Tensor>& Z,
                          const c10::optional<at::Tensor>& rows, const c10::optional<at::Tensor>& cols,
                          const c10::optional<at::Tensor>& meta, int64_t num_rows, const at::Tensor& pair_kind,
                          const at::Tensor& slots, int64_t maxe, const at::Tensor& kind_blocks,
                          const c10::optional<at::Tensor>& perm_out, int64_t t, int64_t num_blocks,
                          const at::Tensor& blocks, const c10::optional<at::Tensor>& w, const at::Tensor& sched,
                          int64_t ngroups, int64_t group_cols, const c10::optional<at::Tensor>& perm_post) {
  require_gpu(fock, "fock");
  TORCH_CHECK_VALUE(fock.scalar_type() == at::kFloat,
                    "Unsupported dtype for the Fock matrix; only float32 is supported.");
  check_fock_args(fock, bdo, off, Z, rows, cols, meta, num_rows, t, blocks, num_blocks,
                  {pair_kind, slots, kind_blocks, perm_out, w, sched, perm_post});
  TORCH_CHECK_VALUE(len(perm_out) < 0 || len(perm_out) == t, "perm_out must have one entry per column");
  TORCH_CHECK_VALUE(len(perm_post) < 0 || len(perm_post) == t, "perm_post must have one entry per column");
  const c10::DeviceGuard guard(fock.device());
  void* st = stream_of(fock);
  at::Tensor out = at::empty({num_rows, t}, fock.options());
  const auto* kb = reinterpret_cast<const uint32_t*>(kind_blocks.data_ptr<int32_t>());
  if (meta.has_value()) {
    check_rc(maloq_fock_to_irreps(fock.data_ptr<float>(), ld, meta->data_ptr<int32_t>(), num_rows,
                                  slots.data_ptr<int32_t>(), static_cast<int>(maxe), kb, out.data_ptr<float>(),
                                  cptr<int32_t>(perm_out), static_cast<int>(t), static_cast<int>(num_blocks),
                                  blocks.data_ptr<int32_t>(), cptr<float>(w), sched.data_ptr<int32_t>(),
                                  static_cast<int>(ngroups), static_cast<int>(group_cols), st),
             "maloq_fock_to_irreps");
  } else {
    TORCH_CHECK_VALUE(off.has_value() && Z.has_value() && rows.has_value() && cols.has_value(),
                      "fock_to_irreps needs a row plan or the pair list");
    check_rc(maloq_fock_to_irreps_pairs(fock.data_ptr<float>(), ld, cptr<int64_t>(bdo), off->data_ptr<int32_t>(),
                                        Z->data_ptr<int32_t>(), rows->data_ptr<int32_t>(), cols->data_ptr<int32_t>(),
                                        num_rows, pair_kind.data_ptr<int32_t>(), slots.data_ptr<int32_t>(),
                                        static_cast<int>(maxe), kb, out.data_ptr<float>(), cptr<int32_t>(perm_out),
                                        static_cast<int>(t), static_cast<int>(num_blocks), blocks.data_ptr<int32_t>(),
                                        cptr<float>(w), sched.data_ptr<int32_t>(), static_cast<int>(ngroups),
                                        static_cast<int>(group_cols), st),
             "maloq_fock_to_irreps_pairs");
  }
  if (!perm_post.has_value()) return out;
  at::Tensor ones = at::ones({t}, fock.options());
  at::Tensor sorted = at::empty_like(out);
  check_rc(maloq_gather_columns(out.data_ptr<float>(), t, num_rows, perm_post->data_ptr<int32_t>(),
                                ones.data_ptr<float>(), static_cast<int>(t), sorted.data_ptr<float>(), t, st),
           "maloq_gather_columns");
  return sorted;
}

// get_H per row, scattered into fock in place (the template's entries only).
// perm_pre: rows of several column groups are un-sorted by a column gather first.
void irreps_to_fock(const at::Tensor& net_out, const at::Tensor& fock, int64_t ld,
                    const c10::optional<at::Tensor>& bdo, const c10::optional<at::Tensor>& off,
                    const c10::optional<at::Tensor>& Z, const c10::optional<at::Tensor>& rows,
                    const c10::optional<at::Tensor>& cols, const c10::optional<at::Tensor>& meta,
                    int64_t num_rows, const at::Tensor& pair_kind, const at::Tensor& slots, int64_t maxe,
                    const at::Tensor& kind_blocks, const c10::optional<at::Tensor>& perm_in, int64_t t,
                    int64_t num_blocks, const at::Tensor& blocks, const c10::optional<at::Tensor>& w,
                    const at::Tensor& sched, int64_t ngroups, int64_t group_cols,
                    const c10::optional<at::Tensor>& perm_pre) {
  require_gpu(fock, "fock");
  require_gpu(net_out, "net_out");
  TORCH_CHECK_VALUE(fock.scalar_type() == at::kFloat && net_out.scalar_type() == at::kFloat,
                    "the Fock matrix and the irreps rows must be float32");
  TORCH_CHECK_VALUE(net_out.dim() == 2 && net_out.size(0) == num_rows && net_out.size(1) == t,
                    "net_out rows must match the atom-pair list");
  check_fock_args(fock, bdo, off, Z, rows, cols, meta, num_rows, t, blocks, num_blocks,
                  {net_out, pair_kind, slots, kind_blocks, perm_in, w, sched, perm_pre});
  TORCH_CHECK_VALUE(len(perm_in) < 0 || len(perm_in) == t, "perm_in must have one entry per column");
  TORCH_CHECK_VALUE(len(perm_pre) < 0 || len(perm_pre) == t, "perm_pre must have one entry per column");
  const c10::DeviceGuard guard(fock.device());
  void* st = stream_of(fock);
  at::Tensor x = net_out.contiguous();
  if (perm_pre.has_value()) {
    at::Tensor ones = at::ones({t}, fock.options());
    at::Tensor u = at::empty_like(x);
    check_rc(maloq_gather_columns(x.data_ptr<float>(), t, num_rows, perm_pre->data_ptr<int32_t>(),
                                  ones.data_ptr<float>(), static_cast<int>(t), u.data_ptr<float>(), t, st),
             "maloq_gather_columns");
    x = u;
  }
  const auto* kb = reinterpret_cast<const uint32_t*>(kind_blocks.data_ptr<int32_t>());
  if (meta.has_value()) {
    check_rc(maloq_irreps_to_fock(x.data_ptr<float>(), cptr<int32_t>(perm_in), fock.data_ptr<float>(), ld,
                                  meta->data_ptr<int32_t>(), num_rows, slots.data_ptr<int32_t>(),
                                  static_cast<int>(maxe), kb, static_cast<int>(t), static_cast<int>(num_blocks),
                                  blocks.data_ptr<int32_t>(), cptr<float>(w), sched.data_ptr<int32_t>(),
                                  static_cast<int>(ngroups), static_cast<int>(group_cols), st),
             "maloq_irreps_to_fock");
  } else {
    TORCH_CHECK_VALUE(off.has_value() && Z.has_value() && rows.has_value() && cols.has_value(),
                      "irreps_to_fock needs a row plan or the pair list");
    check_rc(maloq_irreps_to_fock_pairs(x.data_ptr<float>(), cptr<int32_t>(perm_in), fock.data_ptr<float>(), ld,
                                        cptr<int64_t>(bdo), off->data_ptr<int32_t>(), Z->data_ptr<int32_t>(),
                                        rows->data_ptr<int32_t>(), cols->data_ptr<int32_t>(), num_rows,
                                        pair_kind.data_ptr<int32_t>(), slots.data_ptr<int32_t>(),
                                        static_cast<int>(maxe), kb, static_cast<int>(t), static_cast<int>(num_blocks),
                                        blocks.data_ptr<int32_t>(), cptr<float>(w), sched.data_ptr<int32_t>(),
                                        static_cast<int>(ngroups), static_cast<int>(group_cols), st),
             "maloq_irreps_to_fock_pairs");
  }
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
  m.def("edge_vec_to_wigner(Tensor edge_vec, Tensor jd, int lmax, int seed, bool with_inverse, bool with_eulers) "
        "-> Tensor[]");
  m.def("edge_vec_to_wigner_out(Tensor edge_vec, Tensor jd, int lmax, int seed, Tensor(a!) out) -> ()");
  m.def("rotate(Tensor x, Tensor eulers, Tensor? gather, int lmax, bool inverse) -> Tensor");
  m.def("segment_sum(Tensor msg, Tensor perm, Tensor seg_ptr, int num_segments) -> Tensor");
  m.def("label_transform(Tensor x, Tensor blocks, Tensor? w, Tensor sched, Tensor? perm_in, Tensor? perm_out, "
        "int num_blocks, int ngroups, int group_cols, Tensor? perm_inv) -> Tensor");
  m.def("message_block_fwd(Tensor x, Tensor? rad, Tensor w0, Tensor? b0, Tensor[] wm, Tensor src, Tensor dst, "
        "Tensor seg_ptr, Tensor eulers, int lmax, int mmax, bool gate) -> Tensor[]");
  m.def("message_block_bwd(Tensor grad_out, Tensor? rad, Tensor w0, Tensor[] wm, Tensor bwd_src, "
        "Tensor bwd_dst, Tensor bwd_eidx, Tensor seg_ptr_src, Tensor y, Tensor dk, Tensor? r, Tensor? g, "
        "int num_nodes, int c_in, int lmax, int mmax, bool gate, bool need_rad_grad) -> Tensor[]");
  m.def("basis_row_meta(int ld, Tensor? block_data_offsets, Tensor off, Tensor Z, Tensor rows, Tensor cols, "
        "Tensor pair_kind, int maxe) -> Tensor");
  m.def("fock_to_irreps(Tensor fock, int ld, Tensor? block_data_offsets, Tensor? off, Tensor? Z, Tensor? rows, "
        "Tensor? cols, Tensor? meta, int num_rows, Tensor pair_kind, Tensor slots, int maxe, Tensor kind_blocks, "
        "Tensor? perm_out, int t, int num_blocks, Tensor blocks, Tensor? w, Tensor sched, int ngroups, "
        "int group_cols, Tensor? perm_post) -> Tensor");
  m.def("irreps_to_fock(Tensor net_out, Tensor(a!) fock, int ld, Tensor? block_data_offsets, Tensor? off, "
        "Tensor? Z, Tensor? rows, Tensor? cols, Tensor? meta, int num_rows, Tensor pair_kind, Tensor slots, "
        "int maxe, Tensor kind_blocks, Tensor? perm_in, int t, int num_blocks, Tensor blocks, Tensor? w, "
        "Tensor sched, int ngroups, int group_cols, Tensor? perm_pre) -> ()");
  m.def("_jd_table() -> Tensor", &jd_table);
  m.def("_pack_index(int dtype_code, int lmax, int mmax, bool gate, int c_in, int c_out, int mode) -> Tensor",
        &pack_index_cpu);
}

TORCH_LIBRARY_IMPL(maloq_hip, CUDA, m) {
  m.impl("edge_euler", &edge_euler);
  m.impl("wigner_from_euler", &wigner_from_euler);
  m.impl("edge_vec_to_wigner", &edge_vec_to_wigner);
  m.impl("edge_vec_to_wigner_out", &edge_vec_to_wigner_out);
  m.impl("rotate", &rotate);
  m.impl("segment_sum", &segment_sum);
  m.impl("label_transform", &label_transform);
  m.impl("message_block_fwd", &message_block_fwd);
  m.impl("message_block_bwd", &message_block_bwd);
  m.impl("basis_row_meta", &basis_row_meta);
  m.impl("fock_to_irreps", &fock_to_irreps);
  m.impl("irreps_to_fock", &irreps_to_fock);
}
