"""The benchmark's configurations at their full sizes on the HIP path, checked
against the CPU oracle on a node subset (the oracle runs in fp64 on the
subgraph of the subset's in-edges) and through size-independent properties.

* config 2: 32 x 40 atoms, lmax 4, mmax 2, C 128: fp32 forward and fp32 /
  bf16 backward on the first molecule's nodes;
* config 4: 8 x 150 atoms (8 A cutoff), lmax 6, mmax 2, C 128, gated, bf16:
  forward and backward on a node subset, and bitwise run-to-run determinism of
  the whole graph's forward and gradients;
* config 5: 2000-atom periodic SiO2 cell (6 A cutoff), lmax 4, C 256: bf16
  forward, and bf16 forward and backward through the operators (the
  benchmark's step), on a node subset; the 2s2p1d
  block-sparse basis transform on the whole cell: gather bit-exact against
  the oracle, round trip within 1e-6.

Bars: fp32 within 1e-5 of the output (or gradient) scale, bf16 within 2e-2,
the oracle evaluated on the bf16-rounded inputs and weights.
"""
import math

import numpy as np
import pytest
import torch

from oracle import matrix2labels as om2l
from oracle import message as omsg
from oracle import rotation as orot
from oracle import tensor_decomp as otd

pytestmark = pytest.mark.gpu


def _conv(lmax, mmax, c_in, c_out, gen, gate):
    m_size = [lmax - m + 1 for m in range(mmax + 1)]
    extra = lmax * c_out if gate else 0
    k0 = m_size[0] * c_in
    w0 = torch.randn(m_size[0] * c_out + extra, k0, generator=gen, dtype=torch.float64) / math.sqrt(k0)
    b0 = torch.randn(m_size[0] * c_out + extra, generator=gen, dtype=torch.float64) * 0.1
    wm = [torch.randn(2 * m_size[m] * c_out, m_size[m] * c_in, generator=gen, dtype=torch.float64)
          / math.sqrt(m_size[m] * c_in) / math.sqrt(2) for m in range(1, mmax + 1)]
    return {"w0": w0, "b0": b0, "wm": wm, "c_out": c_out}


def _subset_check(g, nodes, lmax, mmax, C, dtype, gate, device, backward, seed=0, determinism=False,
                  via_ops=False):
    """Run the fused block on the whole graph g and compare the rows of
    ``nodes`` (and, with ``backward``, every gradient of a loss that only
    sees those rows) with the oracle on their in-edges.  ``via_ops``: through
    the registered operators (maloq_hip::message_block_fwd / _bwd), as the
    benchmark's training step runs it."""
    from maloq_amd import message as M
    from maloq_amd import ops as O
    block = O.message_block if via_ops else M.message_block
    from maloq_amd.wigner import extract_euler_angles
    gen = torch.Generator().manual_seed(seed)
    N, E, d = g.num_nodes, g.num_edges, (lmax + 1) ** 2
    q = (lambda t: t.to(dtype).double()) if dtype == torch.bfloat16 else (lambda t: t.float().double())
    x = q(torch.randn(N, d, C, generator=gen, dtype=torch.float64))
    conv = _conv(lmax, mmax, C, C, gen, gate)
    conv = {"w0": q(conv["w0"]), "b0": conv["b0"].float().double(), "wm": [q(w) for w in conv["wm"]], "c_out": C}
    rad = q(torch.rand(E, M.rad_width(lmax, mmax, C), generator=gen, dtype=torch.float64) + 0.5)
    ei = torch.from_numpy(np.stack([g.src, g.dst]))
    eul = extract_euler_angles(torch.from_numpy(g.edge_distance_vec()).float().to(device), seed=seed + 1)
    node_mask = torch.zeros(N, dtype=torch.bool)
    node_mask[torch.as_tensor(nodes)] = True
    sel = node_mask[ei[1]]
    gout = torch.randn(N, d, C, generator=gen, dtype=torch.float64) * node_mask[:, None, None]
    # oracle on the subset's in-edges
    e64 = eul.cpu().double()[sel]
    leaves = [x.clone(), rad[sel].clone(), conv["w0"].clone(), conv["b0"].clone()] + [w.clone() for w in conv["wm"]]
    if backward:
        leaves = [t.requires_grad_() for t in leaves]
    ref = omsg.message_block(leaves[0], ei[:, sel], (e64[:, 0], e64[:, 1], e64[:, 2]), orot.load_jd(), lmax, mmax,
                             {"w0": leaves[2], "b0": leaves[3], "wm": leaves[4:], "c_out": C}, rad=leaves[1],
                             gate=gate)
    if backward:
        (ref * gout).sum().backward()
    # device, whole graph
    plan = M.MessagePlan(ei.to(device), N)

    def run():
        dl = [x.to(device=device, dtype=dtype), plan.sort_edges(rad.to(device=device, dtype=dtype)),
              conv["w0"].float().to(device), conv["b0"].float().to(device)] + [w.float().to(device) for w in conv["wm"]]
        if backward:
            dl = [t.requires_grad_() for t in dl]
        out = block(dl[0], plan, plan.sort_edges(eul), dl[1], dl[2], dl[3], dl[4:], lmax, mmax, gate=gate)
        if backward:
            out.backward(gout.float().to(device))
        torch.cuda.synchronize()
        return out.detach(), [t.grad for t in dl] if backward else []

    out, grads = run()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    idx = torch.as_tensor(nodes)
    got = out.cpu().double()[idx]
    err = (got - ref.detach()[idx]).abs().max().item() / ref.detach()[idx].abs().max().item()
    assert err < tol, f"forward rel err {err}"
    if backward:
        inv = torch.empty_like(plan.perm)
        inv[plan.perm] = torch.arange(E, device=device)
        names = ["x", "rad", "w0", "b0"] + [f"w{m}" for m in range(1, mmax + 1)]
        for n, a, b in zip(names, grads, leaves):
            ga = a[inv].cpu().double()[sel] if n == "rad" else a.cpu().double()
            if n == "rad":
                assert torch.all(a[inv].cpu()[~sel] == 0), "edges outside the subset get no gradient"
            err = (ga - b.grad).abs().max().item() / max(b.grad.abs().max().item(), 1e-30)
            assert err < tol, f"grad {n}: rel err {err}"
    if determinism:
        out2, grads2 = run()
        assert torch.equal(out, out2), "forward not bitwise run-to-run deterministic"
        for a, b in zip(grads, grads2):
            assert torch.equal(a, b), "gradients not bitwise run-to-run deterministic"


@pytest.fixture(scope="module")
def cfg2():
    from maloq_amd.synth import config2_graph
    return config2_graph()


@pytest.fixture(scope="module")
def cfg4():
    from maloq_amd.synth import config4_graph
    return config4_graph()


@pytest.fixture(scope="module")
def cfg5():
    from maloq_amd.synth import config5_graph
    return config5_graph()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config2_first_molecule_fwd_bwd(cfg2, dtype, device):
    print(f"config 2 C=128 dtype={dtype}", flush=True)
    nodes = np.nonzero(cfg2.mol == 0)[0]
    _subset_check(cfg2, nodes, 4, 2, 128, dtype, False, device, backward=True, seed=2)


def test_config4_gated_lmax6_fwd_bwd(cfg4, device):
    print("config 4 lmax=6 C=128 gated bf16", flush=True)
    nodes = np.nonzero(cfg4.mol == 0)[0][:12]
    _subset_check(cfg4, nodes, 6, 2, 128, torch.bfloat16, True, device, backward=True, seed=4, determinism=True)


def test_config5_c256_forward(cfg5, device):
    print("config 5 lmax=4 C=256 bf16", flush=True)
    _subset_check(cfg5, np.arange(0, 2000, 200), 4, 2, 256, torch.bfloat16, False, device, backward=False, seed=5)


def test_config5_c256_fwd_bwd_bf16_operators(cfg5, device):
    """The benchmark's config-5 training step itself (bf16, C = 256, through
    the registered operators: the launches bench.py times) on the whole
    2000-atom cell: the forward rows and every gradient (x, the radial rows,
    the m = 0 weights and bias, the m > 0 weights) of a loss on a node subset,
    against the fp64 oracle on the subset's in-edges."""
    print("config 5 lmax=4 C=256 fwd+bwd bf16 through the operators", flush=True)
    _subset_check(cfg5, np.arange(7, 2000, 250), 4, 2, 256, torch.bfloat16, False, device, backward=True, seed=6,
                  via_ops=True)


@pytest.mark.skip(reason="first run together with a GPU build that faulted the GPU (32-edge forward tiles at three "
                         "workgroups per CU); the faulting case is not identified, so this never-before-run shape stays "
                         "off the GPU until a CPU analysis clears it")
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config5_c256_fwd_bwd(cfg5, dtype, device):
    """The timed config-5 step at its width (C = 256) on the whole 2000-atom
    cell: the forward rows and every gradient (x, the radial rows, the m = 0
    weights and bias, the m > 0 weights) of a loss on a node subset, against
    the fp64 oracle on the subset's in-edges."""
    print(f"config 5 lmax=4 C=256 fwd+bwd dtype={dtype}", flush=True)
    _subset_check(cfg5, np.arange(7, 2000, 250), 4, 2, 256, dtype, False, device, backward=True, seed=6)


def test_config5_block_sparse_transform_full_cell(cfg5, device):
    """2s2p1d (T = 169) on Si and O, every atom pair within 6 A plus on-site
    blocks of the 2000-atom cell, block-list storage (SparseBlockMatrix)."""
    from maloq_amd import tensor_decomp as ptd
    from maloq_amd.basis_transform import HipE3TensorDecomp
    from maloq_amd.matrix2labels import SparseBlockMatrix, hip_single_matrix2label_sparse
    from maloq_amd.synth import atom_pair_rows
    print("config 5 basis transform", flush=True)
    basis = {14: [0, 0, 1, 1, 2], 8: [0, 0, 1, 1, 2]}
    t = ptd.BasisTables(basis)
    base = ptd.e3TensorDecomp(t.req_output_irreps, t.out_js_list, torch.float32, device_torch=device)
    hip = HipE3TensorDecomp(base)
    Z = cfg5.Z
    rows, cols = atom_pair_rows(cfg5.src, cfg5.dst, len(Z))
    off = np.concatenate([[0], np.cumsum(t.orbitals_per_atom(Z))]).astype(np.int32)
    bdo = om2l.block_data_offsets(off, rows, cols)
    rng = np.random.default_rng(0)
    # N(0, 1) exp(-r / 2) blocks; on-site blocks shifted by -10
    vec = {(int(s), int(d)): v for s, d, v in zip(cfg5.src, cfg5.dst, cfg5.vec)}
    data = rng.standard_normal(int(bdo[-1])).astype(np.float32)
    for k, (i, j) in enumerate(zip(rows, cols)):
        sl = slice(int(bdo[k]), int(bdo[k + 1]))
        if i == j:
            n = off[i + 1] - off[i]
            data[sl] = (data[sl].reshape(n, n) - 10.0 * np.eye(n, dtype=np.float32)).reshape(-1)
        else:
            data[sl] *= np.float32(math.exp(-np.linalg.norm(vec[(int(i), int(j))]) / 2))
    T = 169
    ref = np.zeros((len(rows), T), np.float32)
    om2l.single_matrix2label_sparse(t.orbital_template, off, Z, rows, cols, data, bdo, ref, True)
    dd = torch.from_numpy(data).to(device)
    bd = torch.from_numpy(bdo).to(device)
    lab = torch.zeros(len(rows), T, device=device)
    sbm = SparseBlockMatrix(data=dd, block_data_offsets=bd, fock_block_rows=None, fock_block_cols=None,
                            fock_block_offsets=None)
    hip_single_matrix2label_sparse(t.orbital_template, off, Z, rows, cols, lab, None, True, sparse_matrix=sbm,
                                   block_data_offsets=bd)
    assert np.array_equal(lab.cpu().numpy(), ref), "block-sparse gather is not bit-exact"
    irr = hip.fock_to_irreps(dd, off, Z, rows, cols, t.orbital_template, block_data_offsets=bd)
    want = otd.E3TensorDecomp(t.out_js_list).get_net_out(torch.from_numpy(ref[:2000]).double())
    assert (irr[:2000].cpu().double() - want).abs().max() / want.abs().max() < 1e-5
    back = torch.zeros_like(dd)
    hip.irreps_to_fock(irr, back, off, Z, rows, cols, t.orbital_template, block_data_offsets=bd)
    assert (back - dd).abs().max().item() / dd.abs().max().item() < 1e-6
