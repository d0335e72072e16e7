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
//   edgewise_fwd / edgewise_bwd(...)             the two-convolution Edgewise (esen_block.py:146-258),
//                                                node and edge modes, forward and gradients
//   basis_row_meta(...)                          the row plan of the fused Fock transforms
//   fock_to_irreps(fock, ...)                    matrix2label + get_net_out,
//                                                fock_targets_batched.py:335-464
//   irreps_to_fock(net_out, fock!, ...)          get_H + label2matrix (in place),
//                                                splittrainer.py:1172-1233
//   radial_fwd / radial_bwd(...)                 RadialMLP (radial.py:115-142), forward and
//                                                its autograd backward
//   edge_m0_rows, edge_degree_embed[_],          EdgeDegreeEmbedding (embedding.py:17-141):
//   edge_degree_embed_bwd(...)                   m = 0 rows, the embedding (node: in place or a
//                                                copy of x; edge), the gradient wrt the radial rows
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

// Device pointer of an index tensor: of element type T (data_ptr refuses
// another dtype rather than reinterpreting it) and densely packed, since the
// kernels read it as a flat array.
template <class T>
T* iptr(const at::Tensor& t) {
  TORCH_CHECK_VALUE(t.is_contiguous(), "index and table tensors must be contiguous, got sizes ", t.sizes(),
                    " strides ", t.strides());
  return t.data_ptr<T>();
}

// The same for an optional tensor (null if absent).
template <class T>
const T* cptr(const c10::optional<at::Tensor>& t) {
  return t.has_value() ? iptr<T>(*t) : nullptr;
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
    // mode 2: the transposed index, then the forward one (both packings from
    // one launch; the transposed part, which a caller keeps, starts the buffer)
    std::vector<int64_t> idx = pack_index(code, lmax, mmax, gate, c_in, c_out, mode == 2 ? 1 : mode, &tot);
    if (mode == 2) {
      std::vector<int64_t> f0 = pack_index(code, lmax, mmax, gate, c_in, c_out, 0, &tot);
      idx.insert(idx.end(), f0.begin(), f0.end());
    }
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
                        g.defined() ? iptr<int32_t>(g) : nullptr, E, eul.data_ptr<float>(), nullptr,
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
  check_rc(maloq_segment_sum(m.data_ptr<float>(), iptr<int64_t>(p), iptr<int64_t>(s), num_segments,
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
    check_rc(maloq_gather_columns(y.data_ptr<float>(), y.size(1), y.size(0), iptr<int32_t>(src),
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
                                 iptr<int32_t>(blocks), cptr<float>(w), iptr<int32_t>(sched),
                                 static_cast<int>(ngroups), static_cast<int>(group_cols), stream_of(xc)),
           "maloq_label_transform");
  return post ? gather(out, *perm_out) : out;
}

// ----------------------------------------------------------- message block
at::Tensor pack_weights(int code, int64_t lmax, int64_t mmax, bool gate, int64_t c_in, int64_t c_out, int mode,
                        const at::Tensor& w0, at::TensorList wm, at::ScalarType dt);

// Node output and the workspaces the backward reads: [out, y, r, dk, g, wpt]
// (r empty without radial scales, g empty ungated, wpt the backward's
// transposed weight packing with save_tr, else empty); src, dst, seg_ptr and
// eulers are those of the dst-sorted graph plan.
std::vector<at::Tensor> message_block_fwd(const at::Tensor& x, const c10::optional<at::Tensor>& rad,
                                          const at::Tensor& w0, const c10::optional<at::Tensor>& b0,
                                          at::TensorList wm, const at::Tensor& src, const at::Tensor& dst,
                                          const at::Tensor& seg_ptr, const at::Tensor& eulers, int64_t lmax,
                                          int64_t mmax, bool gate, bool save_tr) {
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
  // weights in fragment order; with save_tr also the transposed packing of the
  // backward from the same launch (first in the buffer, returned last)
  at::Tensor wpack, wpt = at::empty({0}, x.options());
  if (save_tr) {
    const at::Tensor p = pack_weights(code, lmax, mmax, gate, c_in, c_out, 2, w0, wm, dt);
    const int64_t nf = maloq_message_wpack_bytes(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                                 static_cast<int>(c_in), static_cast<int>(c_out)) /
                       p.element_size();
    wpt = p.narrow(0, 0, p.numel() - nf);
    wpack = p.narrow(0, p.numel() - nf, nf);
  } else {
    wpack = pack_weights(code, lmax, mmax, gate, c_in, c_out, 0, w0, wm, dt);
  }
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
                             static_cast<int>(c_in), iptr<int32_t>(src), iptr<int32_t>(dst), E,
                             eul.data_ptr<float>(), radc.defined() ? radc.data_ptr() : nullptr, wpack.data_ptr(),
                             bias.defined() ? bias.data_ptr<float>() : nullptr, jd_on(dev), out.data_ptr<float>(),
                             num_nodes, static_cast<int>(c_out), iptr<int64_t>(seg_ptr),
                             parts.data_ptr<float>(), y.data_ptr(), rad.has_value() ? r.data_ptr() : nullptr,
                             dk.data_ptr<float>(), gate ? g.data_ptr() : nullptr, stream_of(xc)),
           "maloq_message_fwd");
  return {out, y, r, dk, g, wpt};
}

// Saved rows of the bf16 weight gradient: rows past E are zero (it reads whole
// 128-edge chunks).
at::Tensor edge_rows(int64_t E, int64_t rows, int64_t c, const at::TensorOptions& opt) {
  const int64_t n = maloq_message_edge_rows(E);
  at::Tensor t = at::empty({n, rows, c}, opt);
  if (n > E) t.narrow(0, E, n - E).zero_();
  return t;
}

// Weights in the kernels' fragment order: mode 0 the forward GEMM's, 1 the
// input gradient's transposed GEMM's, 2 both in one launch (transposed first).
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
  // bytes: the forward packing (c_in -> c_out), the transposed one (c_out -> c_in), or both
  const int64_t fwd_b = maloq_message_wpack_bytes(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                                  static_cast<int>(c_in), static_cast<int>(c_out));
  const int64_t tr_b = maloq_message_wpack_bytes(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                                 static_cast<int>(c_out), static_cast<int>(c_in));
  const int64_t want = mode == 0 ? fwd_b : (mode == 1 ? tr_b : fwd_b + tr_b);
  at::Tensor wpack = at::empty({idx.numel()}, w0.options().dtype(dt));
  TORCH_CHECK(wpack.numel() * wpack.element_size() == want, "packed weight size mismatch");
  check_rc(maloq_message_pack(code, static_cast<int>(sp.size()), sp.data(), sn.data(), iptr<int64_t>(idx),
                              idx.numel(), wpack.data_ptr(), stream_of(w0)),
           "maloq_message_pack");
  return wpack;
}

// Split-K count of the weight gradient over the edges (deterministic: the
// partials are summed in split order).  bf16: 256 x 256 output tiles, one
// workgroup per CU, the most splits that keep every workgroup in one round;
// fp32: 128 x 128 tiles, the count that balances the workgroups over the CUs
// (at most four per CU, the kernel's occupancy; >= 1024 edges per split).
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
    if (ntiles * s > 4 * cus || s > std::max<int64_t>(1, E / 1024)) continue;
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

// Weight and bias gradients of one SO(2) convolution from the saved rows:
// [dW0, db0, dW_1 .. dW_mmax] (fp32, zeros for a graph without edges).  dz the
// output-row gradients [*, d' (+ lmax gated), c_out], y the input rows
// [*, d', c_in], both in the forward's dtype with E valid rows (bf16: the
// padded workspaces of maloq_message_edge_rows).  Split-K over the edges,
// partials summed in split order (deterministic).
std::vector<at::Tensor> weight_grads(const at::Tensor& dz, const at::Tensor& y, int64_t E, int64_t lmax,
                                     int64_t mmax, int64_t c_out, int64_t c_in, bool gate) {
  const auto dt = dz.scalar_type();
  const int code = dtype_code(dt);
  const auto opt32 = dz.options().dtype(at::kFloat);
  const int64_t extra = gate ? lmax * c_out : 0;
  const int kr = maloq_message_kept_rows(static_cast<int>(lmax), static_cast<int>(mmax));
  std::vector<at::Tensor> res;
  if (E == 0) {
    res.push_back(at::zeros({extra + (lmax + 1) * c_out, (lmax + 1) * c_in}, opt32));
    res.push_back(at::zeros({extra + (lmax + 1) * c_out}, opt32));
    for (int64_t m = 1; m <= mmax; ++m) res.push_back(at::zeros({2 * (lmax - m + 1) * c_out, (lmax - m + 1) * c_in}, opt32));
    return res;
  }
  TORCH_CHECK(y.scalar_type() == dt && dz.size(0) >= E && y.size(0) >= E, "weight gradient: bad saved rows");
  if (dt == at::kBFloat16)
    TORCH_CHECK(dz.size(0) >= maloq_message_edge_rows(E) && y.size(0) == dz.size(0),
                "bf16 weight gradient needs the padded workspaces");
  void* st = stream_of(dz);
  const int cus = at::cuda::getDeviceProperties(dz.device().index())->multiProcessorCount;
  const int splits = dw_splits(dt == at::kBFloat16, lmax, mmax, gate, c_out, c_in, E, cus);
  const int64_t dp = maloq_message_dw_partials_floats(static_cast<int>(lmax), static_cast<int>(mmax), gate ? 1 : 0,
                                                      static_cast<int>(c_out), static_cast<int>(c_in), splits);
  at::Tensor dparts = at::empty({dp > 1 ? dp : 1}, opt32);
  at::Tensor dw0 = at::empty({extra + (lmax + 1) * c_out, (lmax + 1) * c_in}, opt32);
  std::vector<at::Tensor> dwm;
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
  at::Tensor db0 = at::empty({extra + (lmax + 1) * c_out}, opt32);
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
  res.push_back(dw0);
  res.push_back(db0);
  for (auto& t : dwm) res.push_back(t);
  return res;
}

// Gradients of message_block_fwd from its saved rows: [grad_x fp32 [N, d, c_in],
// grad_rad (empty unless asked), dW0, db0, dW_1 .. dW_mmax] (fp32).  The
// graph arrives as the plan's source-sorted arrays: bwd_src, bwd_dst,
// bwd_eidx (dst-sorted position of each source-sorted edge), seg_ptr_src;
// dst (optional, the forward's dst-sorted destinations) lets the output
// gradient's rotation read each node's rows once for its consecutive edges.
std::vector<at::Tensor> message_block_bwd(const at::Tensor& grad_out, const c10::optional<at::Tensor>& rad,
                                          const at::Tensor& w0, at::TensorList wm, const at::Tensor& bwd_src,
                                          const at::Tensor& bwd_dst, const at::Tensor& bwd_eidx,
                                          const at::Tensor& seg_ptr_src, const at::Tensor& y, const at::Tensor& dk,
                                          const c10::optional<at::Tensor>& r, const c10::optional<at::Tensor>& g,
                                          int64_t num_nodes, int64_t c_in, int64_t lmax, int64_t mmax, bool gate,
                                          bool need_rad_grad, const c10::optional<at::Tensor>& dst,
                                          const c10::optional<at::Tensor>& wpack_t) {
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
  TORCH_CHECK_VALUE(!dst.has_value() || (dst->scalar_type() == at::kInt && dst->numel() == bwd_src.numel()),
                    "dst must be int32 with one entry per edge");
  TORCH_CHECK_VALUE(seg_ptr_src.numel() == num_nodes + 1, "seg_ptr_src must hold num_nodes + 1 offsets");
  TORCH_CHECK_VALUE(y.dim() == 3 && y.size(0) >= bwd_src.numel() && dk.size(0) >= bwd_src.numel(),
                    "the saved rows must cover every edge");
  same_device(grad_out, {rad, w0, bwd_src, bwd_dst, bwd_eidx, seg_ptr_src, y, dk, r, g, dst});
  for (int64_t m = 0; m < mmax; ++m) same_device(grad_out, {wm[m]});
  const c10::DeviceGuard guard(grad_out.device());
  const int64_t c_out = grad_out.size(2), E = bwd_src.size(0);
  const int kr = maloq_message_kept_rows(static_cast<int>(lmax), static_cast<int>(mmax));
  const auto opt32 = grad_out.options().dtype(at::kFloat);
  void* st = stream_of(grad_out);
  // input gradient (and the radial gradient); the transposed packing saved by
  // the forward (save_tr), or packed here
  at::Tensor wpt;
  if (wpack_t.has_value() && wpack_t->numel() > 0) {
    const int64_t b = maloq_message_wpack_bytes(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                                static_cast<int>(c_out), static_cast<int>(c_in));
    TORCH_CHECK_VALUE(wpack_t->scalar_type() == dt && wpack_t->is_contiguous() &&
                          wpack_t->numel() * wpack_t->element_size() == b && wpack_t->device() == grad_out.device(),
                      "wpack_t is not the transposed packing of these weights");
    wpt = *wpack_t;
  } else {
    wpt = pack_weights(code, lmax, mmax, gate, c_in, c_out, 1, w0, wm, dt);
  }
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
                                gq.data_ptr<float>(), static_cast<int>(c_out), iptr<int32_t>(bwd_dst),
                                iptr<int32_t>(bwd_src), iptr<int32_t>(bwd_eidx), E, dk.data_ptr<float>(),
                                radc.defined() ? radc.data_ptr() : nullptr,
                                grad_rad.numel() ? grad_rad.data_ptr() : nullptr, has_r ? r->data_ptr() : nullptr,
                                wpt.data_ptr(), jd_on(grad_out.device()), gx.data_ptr<float>(), num_nodes,
                                static_cast<int>(c_in), iptr<int64_t>(seg_ptr_src), parts.data_ptr<float>(),
                                dz.data_ptr(), gate ? g->data_ptr() : nullptr, cptr<int32_t>(dst), st),
           "maloq_message_bwd_dx");
  // weight and bias gradients
  std::vector<at::Tensor> wg = weight_grads(dz, y, E, lmax, mmax, c_out, c_in, gate);
  std::vector<at::Tensor> res{gx, grad_rad};
  for (auto& t : wg) res.push_back(t);
  return res;
}

// ------------------------------------------------ two-convolution Edgewise
// The reference's Edgewise (esen_block.py:146-258): message cat(x[src],
// x[dst] [, x_message_edge]), gated SO(2) conv1 (radial scales), conv2, back to
// the global frame and summed per destination node (node mode) or kept per
// edge (edge mode, original edge order).  The graph arrives as the plan's
// dst-sorted arrays (src, dst, seg_ptr) with perm (dst-sorted position ->
// original edge); the frames as dst-sorted Euler triples or as the
// reference's dense wigner [E, d, d] in the original order.  Returns [out, y,
// r, z, dk, g, wp1t, wp2t]: the workspaces the backward reads and, with save,
// both convolutions' transposed weight packings (empty when not kept).
std::vector<at::Tensor> edgewise_fwd(const at::Tensor& x, const c10::optional<at::Tensor>& rad, const at::Tensor& w01,
                                     const c10::optional<at::Tensor>& b01, at::TensorList wm1, const at::Tensor& w02,
                                     const c10::optional<at::Tensor>& b02, at::TensorList wm2, const at::Tensor& src,
                                     const at::Tensor& dst, const at::Tensor& seg_ptr, const at::Tensor& perm,
                                     const c10::optional<at::Tensor>& eulers, const c10::optional<at::Tensor>& wigner,
                                     const c10::optional<at::Tensor>& x_message_edge,
                                     const c10::optional<at::Tensor>& wpack1_in,
                                     const c10::optional<at::Tensor>& wpack2_in, int64_t lmax, int64_t mmax,
                                     bool edge_mode, bool save) {
  const auto dt = x.scalar_type();
  const int code = dtype_code(dt);
  require_gpu(x, "x");
  require_gpu(w01, "w01");
  TORCH_CHECK_VALUE(maloq_message_supported(static_cast<int>(lmax), static_cast<int>(mmax)),
                    "no message kernels for lmax=", lmax, ", mmax=", mmax);
  const int64_t d = (lmax + 1) * (lmax + 1);
  TORCH_CHECK_VALUE(x.dim() == 3 && x.size(1) == d, "x must be [N, (lmax+1)^2, C]");
  TORCH_CHECK_VALUE(eulers.has_value() != wigner.has_value(), "give exactly one of eulers and wigner");
  TORCH_CHECK_VALUE(src.scalar_type() == at::kInt && dst.scalar_type() == at::kInt &&
                        seg_ptr.scalar_type() == at::kLong && perm.scalar_type() == at::kLong,
                    "the plan's src/dst must be int32, seg_ptr and perm int64");
  const int64_t E = src.numel();
  TORCH_CHECK_VALUE(dst.numel() == E && perm.numel() == E, "src, dst and perm must have one entry per edge");
  TORCH_CHECK_VALUE(static_cast<int64_t>(wm1.size()) >= mmax && static_cast<int64_t>(wm2.size()) >= mmax,
                    "wm1 and wm2 need mmax weights each");
  same_device(x, {rad, w01, b01, w02, b02, src, dst, seg_ptr, perm, eulers, wigner, x_message_edge, wpack1_in,
                  wpack2_in});
  for (int64_t m = 0; m < mmax; ++m) same_device(x, {wm1[m], wm2[m]});
  const c10::DeviceGuard guard(x.device());
  const int64_t c_x = x.size(2), c_hidden = w01.size(0) / (2 * lmax + 1), c_out = w02.size(0) / (lmax + 1);
  const int64_t npart = x_message_edge.has_value() ? 3 : 2;
  const int kr = maloq_message_kept_rows(static_cast<int>(lmax), static_cast<int>(mmax));
  const at::Device dev = x.device();
  const auto opt32 = x.options().dtype(at::kFloat);
  void* st = stream_of(x);
  at::Tensor xm;
  if (x_message_edge.has_value()) {
    TORCH_CHECK_VALUE(x_message_edge->dim() == 3 && x_message_edge->size(0) == E && x_message_edge->size(1) == d &&
                          x_message_edge->size(2) == c_x,
                      "x_message_edge must be [E, d, C]");
    xm = x_message_edge->to(dt).contiguous();
  }
  // with save, both packings of each convolution from one launch: the
  // transposed ones are returned for the backward
  // (a caller may pass the forward packings of fixed weights instead)
  auto packs = [&](bool gate, int64_t ci, int64_t co, const at::Tensor& w0, at::TensorList wm,
                   const c10::optional<at::Tensor>& given) {
    const int64_t fb = maloq_message_wpack_bytes(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                                 static_cast<int>(ci), static_cast<int>(co));
    if (given.has_value() && !save) {
      TORCH_CHECK_VALUE(given->scalar_type() == dt && given->is_contiguous() &&
                            given->numel() * given->element_size() == fb,
                        "weight packing of the wrong size");
      return std::make_pair(*given, at::empty({0}, given->options()));
    }
    const at::Tensor p = pack_weights(code, lmax, mmax, gate, ci, co, save ? 2 : 0, w0, wm, dt);
    if (!save) return std::make_pair(p, at::empty({0}, p.options()));
    const int64_t n0 = fb / p.element_size(), n1 = p.numel() - n0;
    return std::make_pair(p.narrow(0, n1, n0), p.narrow(0, 0, n1));
  };
  const auto pk1 = packs(true, npart * c_x, c_hidden, w01, wm1, wpack1_in);
  const auto pk2 = packs(false, c_hidden, c_out, w02, wm2, wpack2_in);
  const at::Tensor& wpack1 = pk1.first;
  const at::Tensor& wpack2 = pk2.first;
  // output rows: nodes, or one per edge (each edge its own segment)
  const int64_t num_nodes = seg_ptr.numel() - 1;
  at::Tensor seg_id, sp = seg_ptr;
  int64_t rows = num_nodes;
  if (edge_mode) {
    rows = E;
    seg_id = at::arange(E, x.options().dtype(at::kInt));
    sp = at::arange(E + 1, x.options().dtype(at::kLong));
  }
  at::Tensor out = at::empty({rows, d, c_out}, opt32);
  const int64_t pf = maloq_message_partials_floats(static_cast<int>(lmax), 0, E, static_cast<int>(c_out));
  at::Tensor parts = at::empty({pf > 1 ? pf : 1}, opt32);
  at::Tensor radc;
  if (rad.has_value()) {
    int64_t rw = 0;
    for (int64_t m = 0; m <= mmax; ++m) rw += (lmax - m + 1) * npart * c_x;
    TORCH_CHECK_VALUE(rad->dim() == 2 && rad->size(0) == E && rad->size(1) == rw,
                      "rad must be [E, sum_m (lmax-m+1) npart C]");
    radc = rad->to(dt).contiguous();
  }
  const int64_t E1 = E > 1 ? E : 1;
  at::Tensor y = save ? edge_rows(E, kr, npart * c_x, x.options()) : at::empty({E1, kr, npart * c_x}, x.options());
  at::Tensor z = save ? edge_rows(E, kr, c_hidden, x.options()) : at::empty({E1, kr, c_hidden}, x.options());
  at::Tensor r = (save && rad.has_value()) ? at::empty({E1, kr, npart * c_x}, x.options()) : at::empty({0}, x.options());
  const int ws = maloq_message_wigner_floats(static_cast<int>(lmax), static_cast<int>(mmax));
  at::Tensor dk = at::empty({E1, ws}, opt32), eul;
  if (wigner.has_value()) {
    TORCH_CHECK_VALUE(wigner->dim() == 3 && wigner->size(0) == E && wigner->size(1) == d && wigner->size(2) == d,
                      "wigner must be [E, d, d]");
    const at::Tensor w = wigner->to(at::kFloat).contiguous();
    if (E > 0)
      check_rc(maloq_message_wigner_rows(static_cast<int>(lmax), static_cast<int>(mmax), w.data_ptr<float>(),
                                         iptr<int64_t>(perm), E, dk.data_ptr<float>(), st),
               "maloq_message_wigner_rows");
  } else {
    TORCH_CHECK_VALUE(eulers->dim() == 2 && eulers->size(0) == E && eulers->size(1) == 3,
                      "eulers must be [E, 3] (dst-sorted)");
    eul = eulers->to(at::kFloat).contiguous();
  }
  at::Tensor g = save ? at::empty({E1, kr + lmax, c_hidden}, x.options()) : at::empty({0}, x.options());
  at::Tensor b1, b2;
  if (b01.has_value()) b1 = b01->to(at::kFloat).contiguous();
  if (b02.has_value()) b2 = b02->to(at::kFloat).contiguous();
  const at::Tensor mrow = xm.defined() ? perm.to(at::kInt).contiguous() : at::Tensor();
  const at::Tensor xc = x.contiguous();
  check_rc(maloq_message_edgewise_fwd(
               code, static_cast<int>(lmax), static_cast<int>(mmax), xc.data_ptr(), static_cast<int>(c_x),
               iptr<int32_t>(src), iptr<int32_t>(dst), seg_id.defined() ? iptr<int32_t>(seg_id) : nullptr,
               E, eul.defined() ? eul.data_ptr<float>() : nullptr, radc.defined() ? radc.data_ptr() : nullptr,
               wpack1.data_ptr(), b1.defined() ? b1.data_ptr<float>() : nullptr, static_cast<int>(c_hidden),
               wpack2.data_ptr(), b2.defined() ? b2.data_ptr<float>() : nullptr, jd_on(dev), out.data_ptr<float>(),
               rows, static_cast<int>(c_out), iptr<int64_t>(sp), parts.data_ptr<float>(), y.data_ptr(),
               r.numel() ? r.data_ptr() : nullptr, dk.data_ptr<float>(), g.numel() ? g.data_ptr() : nullptr,
               z.data_ptr(), xm.defined() ? xm.data_ptr() : nullptr, mrow.defined() ? iptr<int32_t>(mrow) : nullptr,
               st),
           "maloq_message_edgewise_fwd");
  if (edge_mode) {
    // dst-sorted position p holds original edge perm[p]
    at::Tensor per_edge = at::empty_like(out);
    per_edge.index_copy_(0, perm, out);
    out = per_edge;
  }
  return {out, y, r, z, dk, g, pk1.second, pk2.second};
}

// Gradients of edgewise_fwd from its saved rows: [grad_x fp32 [N, d, c_x],
// grad_rad (empty unless asked), grad_x_message_edge (original edge order,
// empty for two-part messages), then for conv1 and conv2 in turn dW0, db0,
// dW_1 .. dW_mmax (fp32; both empty lists' worth of empties when not asked)].
std::vector<at::Tensor> edgewise_bwd(const at::Tensor& grad_out, const c10::optional<at::Tensor>& rad,
                                     const at::Tensor& w01, at::TensorList wm1, const at::Tensor& w02,
                                     at::TensorList wm2, const at::Tensor& dst, const at::Tensor& bwd_src,
                                     const at::Tensor& bwd_eidx, const at::Tensor& perm, const at::Tensor& seg_ptr,
                                     const at::Tensor& seg_ptr_src, const at::Tensor& y,
                                     const c10::optional<at::Tensor>& r, const at::Tensor& z, const at::Tensor& dk,
                                     const at::Tensor& g, const c10::optional<at::Tensor>& wpack1_t,
                                     const c10::optional<at::Tensor>& wpack2_t, int64_t num_nodes, int64_t c_x,
                                     int64_t lmax, int64_t mmax, bool edge_mode, int64_t parts, bool need_rad_grad,
                                     bool need_w1, bool need_w2) {
  const auto dt = y.scalar_type();
  const int code = dtype_code(dt);
  require_gpu(grad_out, "grad_out");
  TORCH_CHECK_VALUE(maloq_message_supported(static_cast<int>(lmax), static_cast<int>(mmax)),
                    "no message kernels for lmax=", lmax, ", mmax=", mmax);
  TORCH_CHECK_VALUE(parts == 2 || parts == 3, "parts must be 2 or 3");
  const int64_t d = (lmax + 1) * (lmax + 1), E = dst.numel();
  TORCH_CHECK_VALUE(dst.scalar_type() == at::kInt && bwd_src.scalar_type() == at::kInt &&
                        bwd_eidx.scalar_type() == at::kInt && perm.scalar_type() == at::kLong &&
                        seg_ptr.scalar_type() == at::kLong && seg_ptr_src.scalar_type() == at::kLong,
                    "plan arrays: dst, bwd_src, bwd_eidx int32; perm, seg_ptr, seg_ptr_src int64");
  TORCH_CHECK_VALUE(bwd_src.numel() == E && bwd_eidx.numel() == E && perm.numel() == E,
                    "the plan arrays must have one entry per edge");
  TORCH_CHECK_VALUE(seg_ptr.numel() == num_nodes + 1 && seg_ptr_src.numel() == num_nodes + 1,
                    "seg_ptr and seg_ptr_src must hold num_nodes + 1 offsets");
  TORCH_CHECK_VALUE(grad_out.dim() == 3 && grad_out.size(0) == (edge_mode ? E : num_nodes) && grad_out.size(1) == d,
                    "grad_out must be [rows, d, C]");
  TORCH_CHECK_VALUE(y.size(0) >= E && z.size(0) >= E && dk.size(0) >= E && g.size(0) >= E,
                    "the saved rows must cover every edge");
  TORCH_CHECK_VALUE(static_cast<int64_t>(wm1.size()) >= mmax && static_cast<int64_t>(wm2.size()) >= mmax,
                    "wm1 and wm2 need mmax weights each");
  same_device(grad_out, {rad, w01, w02, dst, bwd_src, bwd_eidx, perm, seg_ptr, seg_ptr_src, y, r, z, dk, g,
                         wpack1_t, wpack2_t});
  for (int64_t m = 0; m < mmax; ++m) same_device(grad_out, {wm1[m], wm2[m]});
  const c10::DeviceGuard guard(grad_out.device());
  const int64_t c_hidden = w01.size(0) / (2 * lmax + 1);
  const int kr = maloq_message_kept_rows(static_cast<int>(lmax), static_cast<int>(mmax));
  const auto opt32 = grad_out.options().dtype(at::kFloat);
  void* st = stream_of(grad_out);
  // the forward's transposed packings, or packed here
  auto given = [&](const c10::optional<at::Tensor>& p, bool gate, int64_t ci, int64_t co) {
    if (!p.has_value() || p->numel() == 0) return false;
    const int64_t b = maloq_message_wpack_bytes(code, static_cast<int>(lmax), static_cast<int>(mmax), gate,
                                                static_cast<int>(co), static_cast<int>(ci));
    TORCH_CHECK_VALUE(p->scalar_type() == dt && p->is_contiguous() && p->numel() * p->element_size() == b,
                      "transposed weight packing of the wrong size");
    return true;
  };
  const at::Tensor wp1t = given(wpack1_t, true, parts * c_x, c_hidden)
                              ? *wpack1_t : pack_weights(code, lmax, mmax, true, parts * c_x, c_hidden, 1, w01, wm1, dt);
  const at::Tensor wp2t = given(wpack2_t, false, c_hidden, c_x)
                              ? *wpack2_t : pack_weights(code, lmax, mmax, false, c_hidden, c_x, 1, w02, wm2, dt);
  at::Tensor gq = grad_out.to(at::kFloat).contiguous(), grad_row;
  if (edge_mode) {
    gq = gq.index_select(0, perm);   // per-edge gradient rows in dst-sorted order
    grad_row = at::arange(E, grad_out.options().dtype(at::kInt));
  }
  at::Tensor gxs = at::empty({num_nodes, d, c_x}, opt32), gxd = at::empty({num_nodes, d, c_x}, opt32);
  const int64_t E1 = E > 1 ? E : 1;
  at::Tensor gxm, edge_seg;
  if (parts == 3) {
    gxm = at::empty({E1, d, c_x}, opt32);
    edge_seg = at::arange(E, grad_out.options().dtype(at::kInt));
  }
  const int64_t pf = maloq_message_partials_floats(static_cast<int>(lmax), 1, E, static_cast<int>(c_x));
  at::Tensor pbuf = at::empty({pf > 1 ? pf : 1}, opt32);
  at::Tensor radc, grad_rad = at::empty({0}, opt32);
  if (rad.has_value()) {
    radc = rad->to(dt).contiguous();
    if (need_rad_grad) grad_rad = at::empty_like(radc);
  }
  at::Tensor dz2 = edge_rows(E, kr, c_x, y.options()), dz1 = edge_rows(E, kr + lmax, c_hidden, y.options());
  const bool has_r = r.has_value() && r->numel() > 0;
  check_rc(maloq_message_edgewise_bwd_dx(
               code, static_cast<int>(lmax), static_cast<int>(mmax), gq.data_ptr<float>(), static_cast<int>(c_x),
               iptr<int32_t>(dst), grad_row.defined() ? iptr<int32_t>(grad_row) : nullptr,
               iptr<int32_t>(bwd_src), iptr<int32_t>(bwd_eidx), E, dk.data_ptr<float>(),
               radc.defined() ? radc.data_ptr() : nullptr, grad_rad.numel() ? grad_rad.data_ptr() : nullptr,
               has_r ? r->data_ptr() : nullptr, g.data_ptr(), wp1t.data_ptr(), static_cast<int>(c_hidden),
               wp2t.data_ptr(), jd_on(grad_out.device()), gxs.data_ptr<float>(), gxd.data_ptr<float>(), num_nodes,
               iptr<int64_t>(seg_ptr), iptr<int64_t>(seg_ptr_src), pbuf.data_ptr<float>(), dz2.data_ptr(),
               dz1.data_ptr(), edge_seg.defined() ? iptr<int32_t>(edge_seg) : nullptr,
               gxm.defined() ? gxm.data_ptr<float>() : nullptr, st),
           "maloq_message_edgewise_bwd_dx");
  at::Tensor gx = gxs.add_(gxd);
  at::Tensor gm = at::empty({0}, opt32);
  if (parts == 3) {
    gm = at::empty({E, d, c_x}, opt32);
    gm.index_copy_(0, perm, gxm.narrow(0, 0, E));   // dst-sorted position p holds original edge perm[p]
  }
  std::vector<at::Tensor> res{gx, grad_rad, gm};
  auto add = [&](bool need, const at::Tensor& dz, const at::Tensor& rows, int64_t co, int64_t ci, bool gate) {
    if (need) {
      for (auto& t : weight_grads(dz, rows, E, lmax, mmax, co, ci, gate)) res.push_back(t);
    } else {
      for (int64_t k = 0; k < 2 + mmax; ++k) res.push_back(at::empty({0}, opt32));
    }
  };
  add(need_w1, dz1, y, c_hidden, parts * c_x, true);
  add(need_w2, dz2, z, c_x, c_hidden, false);
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
  check_rc(maloq_basis_row_meta(ld, cptr<int64_t>(bdo), iptr<int32_t>(off), iptr<int32_t>(Z),
                                iptr<int32_t>(rows), iptr<int32_t>(cols), R, iptr<int32_t>(pair_kind),
                                static_cast<int>(maxe), iptr<int32_t>(meta), stream_of(rows)),
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
  const auto* kb = reinterpret_cast<const uint32_t*>(iptr<int32_t>(kind_blocks));
  if (meta.has_value()) {
    check_rc(maloq_fock_to_irreps(fock.data_ptr<float>(), ld, iptr<int32_t>(*meta), num_rows,
                                  iptr<int32_t>(slots), static_cast<int>(maxe), kb, out.data_ptr<float>(),
                                  cptr<int32_t>(perm_out), static_cast<int>(t), static_cast<int>(num_blocks),
                                  iptr<int32_t>(blocks), cptr<float>(w), iptr<int32_t>(sched),
                                  static_cast<int>(ngroups), static_cast<int>(group_cols), st),
             "maloq_fock_to_irreps");
  } else {
    TORCH_CHECK_VALUE(off.has_value() && Z.has_value() && rows.has_value() && cols.has_value(),
                      "fock_to_irreps needs a row plan or the pair list");
    check_rc(maloq_fock_to_irreps_pairs(fock.data_ptr<float>(), ld, cptr<int64_t>(bdo), iptr<int32_t>(*off),
                                        iptr<int32_t>(*Z), iptr<int32_t>(*rows), iptr<int32_t>(*cols),
                                        num_rows, iptr<int32_t>(pair_kind), iptr<int32_t>(slots),
                                        static_cast<int>(maxe), kb, out.data_ptr<float>(), cptr<int32_t>(perm_out),
                                        static_cast<int>(t), static_cast<int>(num_blocks), iptr<int32_t>(blocks),
                                        cptr<float>(w), iptr<int32_t>(sched), static_cast<int>(ngroups),
                                        static_cast<int>(group_cols), st),
             "maloq_fock_to_irreps_pairs");
  }
  if (!perm_post.has_value()) return out;
  at::Tensor ones = at::ones({t}, fock.options());
  at::Tensor sorted = at::empty_like(out);
  check_rc(maloq_gather_columns(out.data_ptr<float>(), t, num_rows, iptr<int32_t>(*perm_post),
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
    check_rc(maloq_gather_columns(x.data_ptr<float>(), t, num_rows, iptr<int32_t>(*perm_pre),
                                  ones.data_ptr<float>(), static_cast<int>(t), u.data_ptr<float>(), t, st),
             "maloq_gather_columns");
    x = u;
  }
  const auto* kb = reinterpret_cast<const uint32_t*>(iptr<int32_t>(kind_blocks));
  if (meta.has_value()) {
    check_rc(maloq_irreps_to_fock(x.data_ptr<float>(), cptr<int32_t>(perm_in), fock.data_ptr<float>(), ld,
                                  iptr<int32_t>(*meta), num_rows, iptr<int32_t>(slots),
                                  static_cast<int>(maxe), kb, static_cast<int>(t), static_cast<int>(num_blocks),
                                  iptr<int32_t>(blocks), cptr<float>(w), iptr<int32_t>(sched),
                                  static_cast<int>(ngroups), static_cast<int>(group_cols), st),
             "maloq_irreps_to_fock");
  } else {
    TORCH_CHECK_VALUE(off.has_value() && Z.has_value() && rows.has_value() && cols.has_value(),
                      "irreps_to_fock needs a row plan or the pair list");
    check_rc(maloq_irreps_to_fock_pairs(x.data_ptr<float>(), cptr<int32_t>(perm_in), fock.data_ptr<float>(), ld,
                                        cptr<int64_t>(bdo), iptr<int32_t>(*off), iptr<int32_t>(*Z),
                                        iptr<int32_t>(*rows), iptr<int32_t>(*cols), num_rows,
                                        iptr<int32_t>(pair_kind), iptr<int32_t>(slots),
                                        static_cast<int>(maxe), kb, static_cast<int>(t), static_cast<int>(num_blocks),
                                        iptr<int32_t>(blocks), cptr<float>(w), iptr<int32_t>(sched),
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


// ------------------------------------------------------------ radial MLP
// The fused RadialMLP (radial.py:115-142): hidden layers Linear -> LayerNorm ->
// SiLU, then the output Linear.  params: (W_i, b_i, gamma_i, beta_i) per
// hidden layer, then (W_o, b_o); widths c_0 .. c_H, c_out.
struct RadialShapes {
  int nh;
  std::vector<int> w;
  std::vector<at::Tensor> p;  // fp32, contiguous
  std::vector<const float*> W, b, g, bt;
};

RadialShapes radial_shapes(const at::Tensor& ref, at::TensorList params, at::IntArrayRef widths) {
  RadialShapes r;
  r.nh = static_cast<int>(widths.size()) - 2;
  TORCH_CHECK_VALUE(r.nh >= 1, "RadialMLP needs at least one hidden layer");
  TORCH_CHECK_VALUE(static_cast<int>(params.size()) == 4 * r.nh + 2,
                    "params must be (W, b, LayerNorm weight, LayerNorm bias) per hidden layer, then W_o, b_o");
  for (const auto v : widths) {
    TORCH_CHECK_VALUE(v > 0 && v < (int64_t(1) << 30), "bad width ", v);
    r.w.push_back(static_cast<int>(v));
  }
  TORCH_CHECK_VALUE(maloq_radial_bwd_partials_floats(0, r.nh, r.w.data(), 1) >= 0,
                    "these widths are not supported by the fused radial kernels: ", maloq_last_error());
  for (int i = 0; i < r.nh; ++i) {
    const at::Tensor& W = params[4 * i];
    TORCH_CHECK_VALUE(W.dim() == 2 && W.size(0) == widths[i + 1] && W.size(1) == widths[i],
                      "hidden weight ", i, " must be [", widths[i + 1], ", ", widths[i], "]");
    for (int k = 1; k < 4; ++k)
      TORCH_CHECK_VALUE(params[4 * i + k].numel() == widths[i + 1], "hidden layer ", i, " vectors must have ",
                        widths[i + 1], " entries");
  }
  const at::Tensor& Wo = params[4 * r.nh];
  TORCH_CHECK_VALUE(Wo.dim() == 2 && Wo.size(0) == widths[r.nh + 1] && Wo.size(1) == widths[r.nh],
                    "output weight must be [c_out, c_H]");
  TORCH_CHECK_VALUE(params[4 * r.nh + 1].numel() == widths[r.nh + 1], "output bias must have c_out entries");
  for (const auto& t : params) {
    TORCH_CHECK_VALUE(t.device() == ref.device(), "all tensors must be on ", ref.device());
    r.p.push_back(t.detach().to(at::kFloat).contiguous());
  }
  for (int i = 0; i < r.nh; ++i) {
    r.W.push_back(r.p[4 * i].data_ptr<float>());
    r.b.push_back(r.p[4 * i + 1].data_ptr<float>());
    r.g.push_back(r.p[4 * i + 2].data_ptr<float>());
    r.bt.push_back(r.p[4 * i + 3].data_ptr<float>());
  }
  return r;
}

// [out [E, c_out] (bf16 or fp32), wpack (the packed output weights, read by
// radial_bwd), u_H [E, c_H] (the last hidden activation, empty unless save)].
std::vector<at::Tensor> radial_fwd(const at::Tensor& x, at::TensorList params, at::IntArrayRef widths, double eps,
                                   bool bf16, bool save) {
  require_gpu(x, "x");
  TORCH_CHECK_VALUE(x.dim() == 2 && widths.size() >= 3 && x.size(1) == widths[0], "x must be [E, c_0]");
  const c10::DeviceGuard guard(x.device());
  RadialShapes r = radial_shapes(x, params, widths);
  const int code = bf16 ? 1 : 0;
  const auto dt = bf16 ? at::kBFloat16 : at::kFloat;
  const int64_t E = x.size(0), cH = widths[r.nh], cout = widths[r.nh + 1];
  const at::Tensor xc = x.detach().to(at::kFloat).contiguous();
  at::Tensor wpack = at::empty({maloq_radial_pack_bytes(code, static_cast<int>(cout), static_cast<int>(cH))},
                               x.options().dtype(at::kByte));
  at::Tensor out = at::empty({E, cout}, x.options().dtype(dt));
  at::Tensor sv = save ? at::empty({E, cH}, x.options().dtype(dt)) : at::empty({0}, x.options().dtype(dt));
  check_rc(maloq_radial_fwd(code, r.nh, r.w.data(), xc.data_ptr<float>(), E, r.W.data(), r.b.data(), r.g.data(),
                            r.bt.data(), static_cast<float>(eps), r.p[4 * r.nh].data_ptr<float>(),
                            r.p[4 * r.nh + 1].data_ptr<float>(), wpack.data_ptr(), out.data_ptr(),
                            save ? sv.data_ptr() : nullptr, stream_of(x)),
           "maloq_radial_fwd");
  return {out, wpack, sv};
}

// Gradients from radial_fwd's wpack and u_H: [dx [E, c_0] (empty unless
// need_dx), the hidden layers' gradients flat (per layer dW_i, db_i,
// dgamma_i, dbeta_i), dW_o, db_o], fp32, deterministic.
std::vector<at::Tensor> radial_bwd(const at::Tensor& grad, const at::Tensor& x, const at::Tensor& wpack,
                                   const at::Tensor& save, at::TensorList params, at::IntArrayRef widths, double eps,
                                   bool need_dx) {
  require_gpu(grad, "grad");
  const c10::DeviceGuard guard(grad.device());
  RadialShapes r = radial_shapes(grad, params, widths);
  const bool bf16 = save.scalar_type() == at::kBFloat16;
  const int code = bf16 ? 1 : 0;
  const auto dt = save.scalar_type();
  const int64_t E = x.size(0), c0 = widths[0], cH = widths[r.nh], cout = widths[r.nh + 1];
  TORCH_CHECK_VALUE(x.dim() == 2 && x.size(1) == c0 && grad.dim() == 2 && grad.size(0) == E &&
                        grad.size(1) == cout && save.dim() == 2 && save.size(0) == E && save.size(1) == cH,
                    "x [E, c_0], grad [E, c_out] and the saved u_H [E, c_H] must agree");
  TORCH_CHECK_VALUE(wpack.scalar_type() == at::kByte && wpack.is_contiguous() &&
                        wpack.numel() == maloq_radial_pack_bytes(code, static_cast<int>(cout), static_cast<int>(cH)),
                    "wpack must be radial_fwd's packed weights");
  same_device(grad, {x, wpack, save});
  int64_t n_hid = 0;
  for (int i = 0; i < r.nh; ++i) n_hid += widths[i + 1] * (widths[i] + 3);
  const auto opt32 = grad.options().dtype(at::kFloat);
  if (E == 0)  // no edges: every gradient is zero
    return {need_dx ? at::zeros({E, c0}, opt32) : at::empty({0}, opt32), at::zeros({n_hid}, opt32),
            at::zeros({cout, cH}, opt32), at::zeros({cout}, opt32)};
  at::Tensor dx = need_dx ? at::empty({E, c0}, opt32) : at::empty({0}, opt32);
  at::Tensor gh = at::empty({n_hid}, opt32), dwo = at::empty({cout, cH}, opt32), dbo = at::empty({cout}, opt32);
  const at::Tensor xc = x.detach().to(at::kFloat).contiguous();
  const at::Tensor gq = grad.to(dt).contiguous();
  const at::Tensor sq = save.contiguous();
  const int64_t pf = maloq_radial_bwd_partials_floats(code, r.nh, r.w.data(), E);
  TORCH_CHECK(pf >= 0, "maloq_radial_bwd_partials_floats failed: ", maloq_last_error());
  at::Tensor parts = at::empty({pf > 1 ? pf : 1}, opt32);
  check_rc(maloq_radial_bwd(code, r.nh, r.w.data(), xc.data_ptr<float>(), E, r.W.data(), r.b.data(), r.g.data(),
                            r.bt.data(), static_cast<float>(eps), wpack.data_ptr(), gq.data_ptr(), sq.data_ptr(),
                            need_dx ? dx.data_ptr<float>() : nullptr, parts.data_ptr<float>(), gh.data_ptr<float>(),
                            dwo.data_ptr<float>(), dbo.data_ptr<float>(), stream_of(grad)),
           "maloq_radial_bwd");
  return {dx, gh, dwo, dbo};
}


// ------------------------------------------------------ edge-degree embedding
// EdgeDegreeEmbedding (embedding.py:17-141): the m = 0 rows of every edge's
// Wigner blocks, then the rotated radial embedding summed into x per
// destination node (in place, index_add_ order) or kept per edge.

// rows [E, d] fp32 from exactly one of wigner_inv [E, d, d] and eulers [E, 3].
at::Tensor edge_m0_rows(const c10::optional<at::Tensor>& wigner_inv, const c10::optional<at::Tensor>& eulers,
                        int64_t lmax, int64_t num_edges) {
  TORCH_CHECK_VALUE(wigner_inv.has_value() != eulers.has_value(), "give exactly one of wigner_inv and eulers");
  TORCH_CHECK_VALUE(lmax >= 0 && lmax <= 6 && num_edges >= 0, "lmax must be 0..6");
  const at::Tensor& ref = wigner_inv.has_value() ? *wigner_inv : *eulers;
  require_gpu(ref, wigner_inv.has_value() ? "wigner_inv" : "eulers");
  const int64_t d = (lmax + 1) * (lmax + 1);
  at::Tensor w, e;
  if (wigner_inv.has_value()) {
    TORCH_CHECK_VALUE(wigner_inv->dim() == 3 && wigner_inv->size(0) == num_edges && wigner_inv->size(1) == d &&
                          wigner_inv->size(2) == d,
                      "wigner_inv must be [E, (lmax+1)^2, (lmax+1)^2]");
    w = wigner_inv->to(at::kFloat).contiguous();
  } else {
    TORCH_CHECK_VALUE(eulers->dim() == 2 && eulers->size(0) == num_edges && eulers->size(1) == 3,
                      "eulers must be [E, 3]");
    e = eulers->to(at::kFloat).contiguous();
  }
  const c10::DeviceGuard guard(ref.device());
  at::Tensor rows = at::empty({num_edges, d}, ref.options().dtype(at::kFloat));
  check_rc(maloq_edge_m0_rows(static_cast<int>(lmax), num_edges, w.defined() ? w.data_ptr<float>() : nullptr,
                              e.defined() ? e.data_ptr<float>() : nullptr, e.defined() ? jd_on(ref.device()) : nullptr,
                              rows.data_ptr<float>(), stream_of(ref)),
           "maloq_edge_m0_rows");
  return rows;
}

// Shared checks of the embedding; returns the edge count.
int64_t embed_checks(const at::Tensor& u, const at::Tensor& rows, const at::Tensor& x, int64_t lmax,
                     int64_t channels) {
  require_gpu(u, "u");
  const int64_t E = u.size(0), d = (lmax + 1) * (lmax + 1);
  TORCH_CHECK_VALUE(lmax >= 0 && lmax <= 6 && channels > 0, "lmax must be 0..6 and channels positive");
  TORCH_CHECK_VALUE(u.dim() == 2 && u.size(1) == (lmax + 1) * channels, "u must be [E, (lmax+1) C]");
  TORCH_CHECK_VALUE(rows.dim() == 2 && rows.size(0) == E && rows.size(1) == d && rows.scalar_type() == at::kFloat,
                    "rows must be float32 [E, (lmax+1)^2]");
  TORCH_CHECK_VALUE(x.dim() == 3 && x.size(1) == d && x.size(2) == channels, "x must be [N, (lmax+1)^2, C]");
  dtype_code(u.scalar_type());
  dtype_code(x.scalar_type());
  same_device(u, {rows, x});
  return E;
}

// Node mode, in place on x: x[dst_e] += emb_e / rescale in index_add_ order.
void edge_degree_embed_(at::Tensor& x, const at::Tensor& u, const at::Tensor& rows, const at::Tensor& seg_ptr,
                        const at::Tensor& perm, int64_t lmax, int64_t channels, double rescale) {
  const int64_t E = embed_checks(u, rows, x, lmax, channels);
  TORCH_CHECK_VALUE(x.is_contiguous(), "x must be contiguous for the in-place embedding");
  TORCH_CHECK_VALUE(seg_ptr.scalar_type() == at::kLong && perm.scalar_type() == at::kLong &&
                        seg_ptr.numel() == x.size(0) + 1 && perm.numel() == E,
                    "seg_ptr [N + 1] and perm [E] must be int64 (the dst plan)");
  same_device(u, {seg_ptr, perm});
  const c10::DeviceGuard guard(u.device());
  const at::Tensor uc = u.contiguous();
  check_rc(maloq_edge_degree_embed(dtype_code(u.scalar_type()), dtype_code(x.scalar_type()), static_cast<int>(lmax),
                                   uc.data_ptr(), E, static_cast<int>(channels), rows.data_ptr<float>(),
                                   iptr<int64_t>(seg_ptr), iptr<int64_t>(perm), x.size(0), static_cast<float>(rescale),
                                   x.data_ptr(), nullptr, stream_of(u)),
           "maloq_edge_degree_embed");
}

// The same into a copy of x (node), or the per-edge embedding [E, d, C] in
// the dtype of x (edge mode: x only gives the dtype and shape).
at::Tensor edge_degree_embed(const at::Tensor& x, const at::Tensor& u, const at::Tensor& rows,
                             const c10::optional<at::Tensor>& seg_ptr, const c10::optional<at::Tensor>& perm,
                             int64_t lmax, int64_t channels, double rescale, bool node) {
  const int64_t E = embed_checks(u, rows, x, lmax, channels);
  if (node) {
    TORCH_CHECK_VALUE(seg_ptr.has_value() && perm.has_value(), "node mode needs the dst plan (seg_ptr, perm)");
    at::Tensor out = x.clone(at::MemoryFormat::Contiguous);
    edge_degree_embed_(out, u, rows, *seg_ptr, *perm, lmax, channels, rescale);
    return out;
  }
  const c10::DeviceGuard guard(u.device());
  const int64_t d = (lmax + 1) * (lmax + 1);
  at::Tensor emb = at::empty({E, d, channels}, x.options());
  const at::Tensor uc = u.contiguous();
  check_rc(maloq_edge_degree_embed(dtype_code(u.scalar_type()), dtype_code(x.scalar_type()), static_cast<int>(lmax),
                                   uc.data_ptr(), E, static_cast<int>(channels), rows.data_ptr<float>(), nullptr,
                                   nullptr, 0, static_cast<float>(rescale), x.data_ptr(), emb.data_ptr(), stream_of(u)),
           "maloq_edge_degree_embed");
  return emb;
}

// grad_u [E, (lmax+1) C] fp32 = scale sum_j D[l][j] grad[grad_rows[e]][l^2 + j]
// (node mode: grad_rows = dst, scale = 1 / rescale; edge mode: the identity).
at::Tensor edge_degree_embed_bwd(const at::Tensor& grad, const c10::optional<at::Tensor>& grad_rows,
                                 const at::Tensor& rows, int64_t lmax, int64_t channels, double scale) {
  require_gpu(grad, "grad");
  const int64_t E = rows.size(0), d = (lmax + 1) * (lmax + 1);
  TORCH_CHECK_VALUE(grad.dim() == 3 && grad.size(1) == d && grad.size(2) == channels,
                    "grad must be [*, (lmax+1)^2, C]");
  TORCH_CHECK_VALUE(rows.dim() == 2 && rows.size(1) == d && rows.scalar_type() == at::kFloat,
                    "rows must be float32 [E, (lmax+1)^2]");
  TORCH_CHECK_VALUE(grad_rows.has_value() ? (grad_rows->scalar_type() == at::kLong && grad_rows->numel() == E)
                                          : grad.size(0) == E,
                    "grad_rows must be int64 [E] (or grad [E, d, C] per edge)");
  same_device(grad, {grad_rows, rows});
  const c10::DeviceGuard guard(grad.device());
  const at::Tensor gq = (grad.scalar_type() == at::kBFloat16 ? grad : grad.to(at::kFloat)).contiguous();
  at::Tensor gu = at::empty({E, (lmax + 1) * channels}, grad.options().dtype(at::kFloat));
  check_rc(maloq_edge_degree_embed_bwd(dtype_code(gq.scalar_type()), static_cast<int>(lmax), gq.data_ptr(),
                                       cptr<int64_t>(grad_rows), E, static_cast<int>(channels), rows.data_ptr<float>(),
                                       static_cast<float>(scale), gu.data_ptr<float>(), stream_of(grad)),
           "maloq_edge_degree_embed_bwd");
  return gu;
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
        "Tensor seg_ptr, Tensor eulers, int lmax, int mmax, bool gate, bool save_tr=False) -> Tensor[]");
  m.def("message_block_bwd(Tensor grad_out, Tensor? rad, Tensor w0, Tensor[] wm, Tensor bwd_src, "
        "Tensor bwd_dst, Tensor bwd_eidx, Tensor seg_ptr_src, Tensor y, Tensor dk, Tensor? r, Tensor? g, "
        "int num_nodes, int c_in, int lmax, int mmax, bool gate, bool need_rad_grad, Tensor? dst=None, "
        "Tensor? wpack_t=None) -> Tensor[]");
  m.def("edgewise_fwd(Tensor x, Tensor? rad, Tensor w01, Tensor? b01, Tensor[] wm1, Tensor w02, Tensor? b02, "
        "Tensor[] wm2, Tensor src, Tensor dst, Tensor seg_ptr, Tensor perm, Tensor? eulers, Tensor? wigner, "
        "Tensor? x_message_edge, Tensor? wpack1, Tensor? wpack2, int lmax, int mmax, bool edge_mode, bool save) "
        "-> Tensor[]");
  m.def("edgewise_bwd(Tensor grad_out, Tensor? rad, Tensor w01, Tensor[] wm1, Tensor w02, Tensor[] wm2, "
        "Tensor dst, Tensor bwd_src, Tensor bwd_eidx, Tensor perm, Tensor seg_ptr, Tensor seg_ptr_src, Tensor y, "
        "Tensor? r, Tensor z, Tensor dk, Tensor g, Tensor? wpack1_t, Tensor? wpack2_t, int num_nodes, int c_x, "
        "int lmax, int mmax, bool edge_mode, int parts, bool need_rad_grad, bool need_w1, bool need_w2) -> Tensor[]");
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
  m.def("radial_fwd(Tensor x, Tensor[] params, int[] widths, float eps, bool bf16, bool save) -> Tensor[]");
  m.def("radial_bwd(Tensor grad, Tensor x, Tensor wpack, Tensor save, Tensor[] params, int[] widths, float eps, "
        "bool need_dx) -> Tensor[]");
  m.def("edge_m0_rows(Tensor? wigner_inv, Tensor? eulers, int lmax, int num_edges) -> Tensor");
  m.def("edge_degree_embed(Tensor x, Tensor u, Tensor rows, Tensor? seg_ptr, Tensor? perm, int lmax, int channels, "
        "float rescale, bool node) -> Tensor");
  m.def("edge_degree_embed_(Tensor(a!) x, Tensor u, Tensor rows, Tensor seg_ptr, Tensor perm, int lmax, "
        "int channels, float rescale) -> ()");
  m.def("edge_degree_embed_bwd(Tensor grad, Tensor? grad_rows, Tensor rows, int lmax, int channels, float scale) "
        "-> Tensor");
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
  m.impl("edgewise_fwd", &edgewise_fwd);
  m.impl("edgewise_bwd", &edgewise_bwd);
  m.impl("basis_row_meta", &basis_row_meta);
  m.impl("fock_to_irreps", &fock_to_irreps);
  m.impl("irreps_to_fock", &irreps_to_fock);
  m.impl("radial_fwd", &radial_fwd);
  m.impl("radial_bwd", &radial_bwd);
  m.impl("edge_m0_rows", &edge_m0_rows);
  m.impl("edge_degree_embed", &edge_degree_embed);
  m.impl("edge_degree_embed_", &edge_degree_embed_);
  m.impl("edge_degree_embed_bwd", &edge_degree_embed_bwd);
}
