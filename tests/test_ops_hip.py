"""The registered PyTorch custom ops (namespace maloq_hip): schema, fake
(meta) implementations and autograd registration checked by
torch.library.opcheck; a whole rotate-in / rotate-out chain and an Edgewise
forward + backward compiled with torch.compile(fullgraph=True) (no graph
break: every op has a fake implementation); and each op against the
module-level path it wraps, bitwise."""
import math

import numpy as np
import pytest
import torch


def test_ops_are_registered():
    import maloq_amd.ops  # noqa: F401
    for name in ("edge_euler", "wigner_from_euler", "edge_vec_to_wigner", "edge_vec_to_wigner_out", "rotate", "segment_sum", "label_transform",
                 "message_block_fwd", "message_block_bwd", "basis_row_meta", "fock_to_irreps", "irreps_to_fock"):
        assert hasattr(torch.ops.maloq_hip, name), name


@pytest.mark.gpu
def test_opcheck(device):
    from maloq_amd import ops
    gen = torch.Generator().manual_seed(0)
    vec = torch.randn(50, 3, generator=gen).to(device)
    torch.library.opcheck(ops.edge_euler, (vec, 7), test_utils=("test_schema", "test_faketensor"))
    eul = ops.edge_euler(vec, 7)
    torch.library.opcheck(ops.wigner_from_euler, (eul, 3, False), test_utils=("test_schema", "test_faketensor"))
    from maloq_amd.wigner import _packed_jd
    jd = _packed_jd(None, 3, vec.device)
    for inv, with_e in ((False, False), (True, True)):
        torch.library.opcheck(ops.edge_vec_to_wigner, (vec, jd, 3, 7, inv, with_e),
                              test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(ops.edge_vec_to_wigner_out, (vec, jd, 3, 7, torch.zeros(50, 16, 16, device=device)),
                          test_utils=("test_schema", "test_faketensor"))
    x = torch.randn(9, 16, 8, generator=gen).to(device).requires_grad_()
    gather = torch.randint(0, 9, (50,), generator=gen).to(device)
    torch.library.opcheck(ops.rotate, (x, eul, gather, 3, False),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
    msg = torch.randn(50, 4, 8, generator=gen).to(device)
    perm = torch.sort(gather, stable=True).indices
    seg = torch.cat([torch.zeros(1, dtype=torch.int64, device=device),
                     torch.cumsum(torch.bincount(gather, minlength=9), 0)])
    torch.library.opcheck(ops.segment_sum, (msg, perm, seg, 9), test_utils=("test_schema", "test_faketensor"))
    # the fused block's forward: its fake gives the saved rows the library's padding
    from maloq_amd import message as M
    L, C, E, N = 2, 32, 50, 9
    ei = torch.stack([torch.randint(0, N, (E,), generator=gen), gather.cpu()]).to(device)
    plan = M.MessagePlan(ei, N)
    xm = torch.randn(N, (L + 1) ** 2, C, generator=gen).to(device)
    w0 = torch.randn((L + 1) * C + L * C, (L + 1) * C, generator=gen).to(device)
    b0 = torch.randn((L + 1) * C + L * C, generator=gen).to(device)
    wm = [torch.randn(2 * (L - m + 1) * C, (L - m + 1) * C, generator=gen).to(device) for m in (1, 2)]
    rad = torch.rand(E, M.rad_width(L, L, C), generator=gen).to(device)
    for gate in (False, True):
        w0g, b0g = (w0, b0) if gate else (w0[:(L + 1) * C], b0[:(L + 1) * C])
        for save_tr in (False, True):  # with save_tr the backward's weight packing comes along
            args = (xm, rad, w0g, b0g, wm, plan.src, plan.dst, plan.seg_ptr, plan.sort_edges(eul), L, L, gate,
                    save_tr)
            torch.library.opcheck(ops.message_block_fwd, args, test_utils=("test_schema", "test_faketensor"))
            out, y, r, dk, g, wpt = ops.message_block_fwd(*args)
            assert (wpt.numel() > 0) == save_tr
            gout = torch.randn(out.shape, generator=gen).to(device)
            torch.library.opcheck(ops.message_block_bwd,
                                  (gout, rad, w0g, wm, plan.bwd_src, plan.bwd_dst, plan.bwd_eidx, plan.seg_ptr_src,
                                   y, dk, r, g if gate else None, N, C, L, L, gate, True, plan.dst,
                                   wpt if save_tr else None),
                                  test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
def test_compiled_rotation_chain_has_no_graph_break(device):
    from maloq_amd import ops
    from maloq_amd.rotate import rotate
    gen = torch.Generator().manual_seed(1)
    vec = torch.randn(300, 3, generator=gen).to(device)
    x = torch.randn(40, 25, 32, generator=gen).to(device)
    src = torch.randint(0, 40, (300,), generator=gen).to(device)

    def chain(vec, x, src):
        eul = torch.ops.maloq_hip.edge_euler(vec, 3)
        y = torch.ops.maloq_hip.rotate(x, eul, src, 4, False)
        return torch.ops.maloq_hip.rotate(y * 2.0, eul, None, 4, True)

    compiled = torch.compile(chain, backend="aot_eager", fullgraph=True)
    got = compiled(vec, x, src)
    from maloq_amd.wigner import extract_euler_angles
    eul = extract_euler_angles(vec, 3)
    want = rotate(rotate(x, 4, eulers=eul, gather=src) * 2.0, 4, eulers=eul, inverse=True)
    assert torch.equal(got, want)
    assert (got - 2.0 * x[src]).abs().max().item() / x.abs().max().item() < 1e-5


@pytest.mark.gpu
def test_message_block_op_matches_module_path(device):
    from maloq_amd import message as M
    from maloq_amd import ops
    from maloq_amd.wigner import extract_euler_angles
    lmax, mmax, C, N, E = 4, 2, 32, 30, 400
    gen = torch.Generator().manual_seed(2)
    ei = torch.stack([torch.randint(0, N, (E,), generator=gen), torch.randint(0, N, (E,), generator=gen)])
    plan = M.MessagePlan(ei.to(device), N)
    eul = plan.sort_edges(extract_euler_angles(torch.randn(E, 3, generator=gen).to(device), seed=1))
    x0 = torch.randn(N, 25, C, generator=gen).to(device)
    rad0 = (torch.rand(E, M.rad_width(lmax, mmax, C), generator=gen) + 0.5).to(device)
    w00 = (torch.randn(5 * C, 5 * C, generator=gen) / math.sqrt(5 * C)).to(device)
    b00 = torch.randn(5 * C, generator=gen).to(device) * 0.1
    wm0 = [(torch.randn(2 * (5 - m) * C, (5 - m) * C, generator=gen) / math.sqrt((5 - m) * C)).to(device)
           for m in (1, 2)]
    gout = torch.randn(N, 25, C, generator=gen).to(device)
    res = []
    for fn in (M.message_block, ops.message_block):
        leaves = [t.clone().requires_grad_() for t in [x0, rad0, w00, b00] + wm0]
        out = fn(leaves[0], plan, eul, leaves[1], leaves[2], leaves[3], leaves[4:], lmax, mmax)
        out.backward(gout)
        res.append([out.detach()] + [t.grad for t in leaves])
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("basis,if_sort", [({1: [0, 0, 1], 6: [0, 0, 0, 1, 1, 2]}, False),
                                           ({1: [0, 0, 0, 1, 1], 8: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 1, 2]},
                                            True)])
def test_label_transform_op_matches_decomp(basis, if_sort, device):
    """The op equals the decomposition's methods bit for bit, forward and
    gradient, for one column group and for sorted rows of several groups (the
    def2-TZVPD H/O width, 1600 columns); opcheck covers its schema and fake."""
    from maloq_amd import ops
    from maloq_amd import tensor_decomp as ptd
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t = ptd.BasisTables(basis)
    irreps = t.simplified_irreps if if_sort else t.req_output_irreps
    hip = HipE3TensorDecomp(ptd.e3TensorDecomp(irreps, t.out_js_list, torch.float32, if_sort=if_sort,
                                               device_torch=device))
    assert (hip.ngroups > 1) == if_sort
    gen = torch.Generator().manual_seed(3)
    H = torch.randn(77, hip.total_h_dim, generator=gen).to(device)
    assert torch.equal(ops.get_net_out(hip, H), hip.get_net_out(H))
    y = torch.randn(77, hip.total_in_dim, generator=gen).to(device).requires_grad_()
    y2 = y.detach().clone().requires_grad_()
    a, b = ops.get_H(hip, y), hip.get_H(y2)
    assert torch.equal(a, b)
    g = torch.randn_like(a)
    a.backward(g)
    b.backward(g)
    assert torch.equal(y.grad, y2.grad)
    torch.library.opcheck(ops.label_transform, (H, hip._blocks_fwd, hip._wk_fwd, hip._sched, None, hip._perm)
                          + ops._layout(hip), test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
def test_fused_fock_ops_opcheck(device):
    """Schema and fake implementations of the fused Fock operators, on the
    arguments HipE3TensorDecomp passes (a SiO2 block list, with and without a
    row plan); the in-place irreps_to_fock is checked as a mutating op."""
    from maloq_amd import ops
    from maloq_amd import tensor_decomp as ptd
    from maloq_amd.basis_transform import HipE3TensorDecomp
    from maloq_amd.synth import atom_pair_rows, radius_graph, sio2_cell
    from oracle import matrix2labels as om2l
    t = ptd.BasisTables({8: [0, 0, 1, 1, 2], 14: [0, 0, 1, 1, 2]})
    hip = HipE3TensorDecomp(ptd.e3TensorDecomp(t.req_output_irreps, t.out_js_list, torch.float32,
                                               device_torch=device))
    Z, pos, L = sio2_cell(n_atoms=30, seed=2, iters=50)
    src, dst, _ = radius_graph(pos, 5.0, cell=L)
    rows, cols = atom_pair_rows(src, dst, len(Z))
    off = np.concatenate([[0], np.cumsum(t.orbitals_per_atom(Z))]).astype(np.int32)
    bdo = om2l.block_data_offsets(off, rows, cols)
    gen = torch.Generator().manual_seed(4)
    data = torch.randn(int(bdo[-1]), generator=gen).to(device)
    bd = torch.from_numpy(bdo).to(device)
    dev_i32 = lambda a: torch.as_tensor(np.asarray(a, np.int32), device=device)
    o, z, r, c = (dev_i32(a) for a in (off, Z, rows, cols))
    tabs = hip._template_tables(t.orbital_template)
    R = len(rows)
    torch.library.opcheck(ops.basis_row_meta, (0, bd, o, z, r, c, tabs["pair_kind"], tabs["maxe"]),
                          test_utils=("test_schema", "test_faketensor"))
    meta = ops.basis_row_meta(0, bd, o, z, r, c, tabs["pair_kind"], tabs["maxe"])
    common = (tabs["pair_kind"], tabs["slots"], tabs["maxe"], tabs["kind_blocks"])
    tail = (hip.num_blocks, hip._blocks_fwd, hip._wk_fwd, hip._sched, hip.ngroups, hip.group_cols, None)
    for m in (None, meta):
        pairs = (bd, o, z, r, c) if m is None else (None, None, None, None, None)
        torch.library.opcheck(ops.fock_to_irreps, (data, 0) + pairs + (m, R) + common + (None, hip.total_in_dim)
                              + tail, test_utils=("test_schema", "test_faketensor"))
    lab = hip.fock_to_irreps(data, off, Z, rows, cols, t.orbital_template, block_data_offsets=bd)
    back = torch.zeros_like(data)
    torch.library.opcheck(ops.irreps_to_fock, (lab, back, 0, bd, o, z, r, c, None, R) + common
                          + (None, hip.total_in_dim, hip.num_blocks, hip._blocks_inv, hip._wk_inv, hip._sched,
                             hip.ngroups, hip.group_cols, None),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
def test_operators_refuse_inconsistent_arguments(device):
    """The operators take raw device pointers into the kernels, so shapes that
    would read or write past a buffer are refused on the host (ValueError)
    before any launch."""
    from maloq_amd import ops
    msg = torch.zeros(10, 4, device=device)
    perm = torch.arange(10, device=device)
    with pytest.raises(ValueError, match="seg_ptr"):
        ops.segment_sum(msg, perm, torch.zeros(3, dtype=torch.int64, device=device), 5)
    with pytest.raises(ValueError, match="perm"):
        ops.segment_sum(msg, perm[:4], torch.zeros(6, dtype=torch.int64, device=device), 5)
    x = torch.zeros(3, 25, device=device)
    blocks = torch.zeros(2, 4, dtype=torch.int32, device=device)
    sched = torch.zeros(8, dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="column permutations"):
        ops.label_transform(x, blocks, None, sched, torch.zeros(24, dtype=torch.int32, device=device), None,
                            2, 1, 25, None)
    with pytest.raises(ValueError, match="blocks"):
        ops.label_transform(x, blocks, None, sched, None, None, 3, 1, 25, None)
    fock = torch.zeros(100, device=device)
    i32 = torch.zeros(4, dtype=torch.int32, device=device)
    meta = torch.zeros(2, 4, dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="row plan"):
        ops.fock_to_irreps(fock, 0, None, None, None, None, None, meta, 5, i32, i32, 1, i32, None, 25, 2, blocks,
                           None, sched, 1, 25, None)
    with pytest.raises(ValueError, match="rows and cols"):
        ops.basis_row_meta(0, None, i32, i32, i32, i32[:2], i32, 1)
    # index tensors are read as flat arrays: a strided one is refused, not misread
    with pytest.raises(ValueError, match="contiguous"):
        ops.basis_row_meta(0, None, i32, i32, torch.zeros(8, dtype=torch.int32, device=device)[::2], i32, i32, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("mode,parts", [("node", 2), ("edge", 3)])
def test_edgewise_ops_opcheck(mode, parts, device):
    """Schema and fake implementations of the two-convolution Edgewise
    operators on the arguments maloq_amd.message passes."""
    from maloq_amd import message as M
    from maloq_amd import ops
    from maloq_amd.wigner import extract_euler_angles
    L, C, H, N, E = 2, 32, 32, 9, 40
    gen = torch.Generator().manual_seed(9)
    ei = torch.stack([torch.randint(0, N, (E,), generator=gen), torch.randint(0, N, (E,), generator=gen)]).to(device)
    plan = M.MessagePlan(ei, N)
    eul = plan.sort_edges(extract_euler_angles(torch.randn(E, 3, generator=gen).to(device), seed=1))
    x = torch.randn(N, 9, C, generator=gen).to(device)
    xm = torch.randn(E, 9, C, generator=gen).to(device) if parts == 3 else None
    w01 = torch.randn(5 * H, 3 * parts * C, generator=gen).to(device) / 10
    b01 = torch.randn(5 * H, generator=gen).to(device)
    wm1 = [torch.randn(2 * (3 - m) * H, (3 - m) * parts * C, generator=gen).to(device) / 10 for m in (1, 2)]
    w02 = torch.randn(3 * C, 3 * H, generator=gen).to(device) / 10
    b02 = torch.randn(3 * C, generator=gen).to(device)
    wm2 = [torch.randn(2 * (3 - m) * C, (3 - m) * H, generator=gen).to(device) / 10 for m in (1, 2)]
    rad = torch.rand(E, M.rad_width(L, L, parts * C), generator=gen).to(device) + 0.5
    args = (x, rad, w01, b01, wm1, w02, b02, wm2, plan.src, plan.dst, plan.seg_ptr, plan.perm, eul, None, xm, None,
            None, L, L, mode == "edge", True)
    torch.library.opcheck(ops.edgewise_fwd, args, test_utils=("test_schema", "test_faketensor"))
    out, y, r, z, dk, g, wp1t, wp2t = ops.edgewise_fwd(*args)
    gout = torch.randn(out.shape, generator=gen).to(device)
    torch.library.opcheck(ops.edgewise_bwd, (gout, rad, w01, wm1, w02, wm2, plan.dst, plan.bwd_src, plan.bwd_eidx,
                                             plan.perm, plan.seg_ptr, plan.seg_ptr_src, y, r, z, dk, g, wp1t, wp2t, N,
                                             C, L, L, mode == "edge", parts, True, True, True),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
def test_compiled_edgewise_forward_and_backward_have_no_graph_break(device):
    """maloq_hip::edgewise_fwd and edgewise_bwd traced together by
    torch.compile(fullgraph=True): the fake implementations carry every shape
    the graph needs (the saved workspaces included), and the compiled step
    gives the eager result bit for bit."""
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    L, C, H, N, E = 2, 32, 32, 9, 40
    gen = torch.Generator().manual_seed(11)
    ei = torch.stack([torch.randint(0, N, (E,), generator=gen), torch.randint(0, N, (E,), generator=gen)]).to(device)
    plan = M.MessagePlan(ei, N)
    eul = plan.sort_edges(extract_euler_angles(torch.randn(E, 3, generator=gen).to(device), seed=1))
    x = torch.randn(N, 9, C, generator=gen).to(device)
    w01 = torch.randn(5 * H, 3 * 2 * C, generator=gen).to(device) / 10
    b01 = torch.randn(5 * H, generator=gen).to(device)
    wm1 = [torch.randn(2 * (3 - m) * H, (3 - m) * 2 * C, generator=gen).to(device) / 10 for m in (1, 2)]
    w02 = torch.randn(3 * C, 3 * H, generator=gen).to(device) / 10
    b02 = torch.randn(3 * C, generator=gen).to(device)
    wm2 = [torch.randn(2 * (3 - m) * C, (3 - m) * H, generator=gen).to(device) / 10 for m in (1, 2)]
    rad = torch.rand(E, M.rad_width(L, L, 2 * C), generator=gen).to(device) + 0.5
    gout = torch.randn(N, 9, C, generator=gen).to(device)

    def step(x, rad, gout):
        out, y, r, z, dk, g, wp1t, wp2t = torch.ops.maloq_hip.edgewise_fwd(
            x, rad, w01, b01, wm1, w02, b02, wm2, plan.src, plan.dst, plan.seg_ptr, plan.perm, eul, None, None,
            None, None, L, L, False, True)
        res = torch.ops.maloq_hip.edgewise_bwd(
            gout, rad, w01, wm1, w02, wm2, plan.dst, plan.bwd_src, plan.bwd_eidx, plan.perm, plan.seg_ptr,
            plan.seg_ptr_src, y, r, z, dk, g, wp1t, wp2t, N, C, L, L, False, 2, True, True, True)
        return [out] + list(res)

    want = step(x, rad, gout)
    got = torch.compile(step, backend="aot_eager", fullgraph=True)(x, rad, gout)
    assert len(got) == len(want)
    for a, b in zip(got, want):
        assert a.shape == b.shape and torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("bf16", [False, True])
def test_radial_ops_opcheck(bf16, device):
    """Schema and fake implementations of maloq_hip::radial_fwd / radial_bwd
    on the arguments maloq_amd.radial passes."""
    from maloq_amd import ops
    from maloq_amd.radial import RadialMLP
    torch.manual_seed(3)
    widths = [8, 64, 64, 128]
    mod = RadialMLP(widths).to(device)
    params = [p.detach() for li, ln in zip([m for m in mod.net if isinstance(m, torch.nn.Linear)][:-1],
                                           [m for m in mod.net if isinstance(m, torch.nn.LayerNorm)])
              for p in (li.weight, li.bias, ln.weight, ln.bias)]
    lo = [m for m in mod.net if isinstance(m, torch.nn.Linear)][-1]
    params += [lo.weight.detach(), lo.bias.detach()]
    x = torch.randn(150, 8, device=device)
    eps = [m for m in mod.net if isinstance(m, torch.nn.LayerNorm)][0].eps
    args = (x, params, widths, eps, bf16, True)
    torch.library.opcheck(ops.radial_fwd, args, test_utils=("test_schema", "test_faketensor"))
    out, wpack, save = ops.radial_fwd(*args)
    g = torch.randn(out.shape, device=device).to(out.dtype)
    torch.library.opcheck(ops.radial_bwd, (g, x, wpack, save, params, widths, eps, True),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["node", "edge"])
def test_embedding_ops_opcheck(mode, device):
    """Schema and fake implementations of the EdgeDegreeEmbedding operators on
    the arguments maloq_amd.embedding passes, and the in-place node variant
    equal to the functional one."""
    from maloq_amd import ops
    from maloq_amd.message import MessagePlan
    from maloq_amd.wigner import extract_euler_angles
    torch.manual_seed(4)
    lmax, C, N, E = 4, 32, 40, 300
    ei = torch.randint(0, N, (2, E), device=device)
    plan = MessagePlan(ei, N)
    eul = extract_euler_angles(torch.randn(E, 3, device=device), seed=2)
    torch.library.opcheck(ops.edge_m0_rows, (None, eul, lmax, E), test_utils=("test_schema", "test_faketensor"))
    rows = ops.edge_m0_rows(None, eul, lmax, E)
    u = torch.randn(E, (lmax + 1) * C, device=device)
    x = torch.randn(N, (lmax + 1) ** 2, C, device=device)
    node = mode == "node"
    args = (x, u, rows, plan.seg_ptr if node else None, plan.perm if node else None, lmax, C, 0.5, node)
    torch.library.opcheck(ops.edge_degree_embed, args, test_utils=("test_schema", "test_faketensor"))
    out = ops.edge_degree_embed(*args)
    if node:
        xi = x.clone()
        torch.library.opcheck(ops.edge_degree_embed_, (xi.clone(), u, rows, plan.seg_ptr, plan.perm, lmax, C, 0.5),
                              test_utils=("test_schema", "test_faketensor"))
        ops.edge_degree_embed_(xi, u, rows, plan.seg_ptr, plan.perm, lmax, C, 0.5)
        assert torch.equal(xi, out)
    g = torch.randn(out.shape, device=device)
    grows = ei[1].contiguous() if node else None
    torch.library.opcheck(ops.edge_degree_embed_bwd, (g, grows, rows, lmax, C, 2.0 if node else 1.0),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
def test_embedding_ops_refuse_bad_arguments(device):
    """The embedding operators raise ValueError (TORCH_CHECK_VALUE) on the
    argument errors the C++ layer checks, before any launch."""
    from maloq_amd import ops
    lmax, C, N, E = 2, 16, 5, 7
    d = (lmax + 1) ** 2
    u = torch.randn(E, (lmax + 1) * C, device=device)
    x = torch.randn(N, d, C, device=device)
    rows = torch.randn(E, d, device=device)
    seg = torch.zeros(N + 1, dtype=torch.long, device=device)
    perm = torch.arange(E, device=device)
    with pytest.raises(ValueError):  # both Wigner sources
        ops.edge_m0_rows(torch.zeros(E, d, d, device=device), torch.zeros(E, 3, device=device), lmax, E)
    with pytest.raises(ValueError):  # rows in bf16
        ops.edge_degree_embed(x, u, rows.bfloat16(), seg, perm, lmax, C, 1.0, True)
    with pytest.raises(ValueError):  # node mode without the dst plan
        ops.edge_degree_embed(x, u, rows, None, None, lmax, C, 1.0, True)
    with pytest.raises(ValueError):  # u of the wrong width
        ops.edge_degree_embed(x, u[:, :-1], rows, seg, perm, lmax, C, 1.0, True)
    with pytest.raises(ValueError):  # seg_ptr of the wrong length
        ops.edge_degree_embed_(x, u, rows, seg[:-1], perm, lmax, C, 1.0)
    with pytest.raises(ValueError):  # grad_rows of the wrong length
        ops.edge_degree_embed_bwd(x, perm[:-1], rows, lmax, C, 1.0)
