"""GPU parity of the fused message block against the CPU oracle
(oracle.message.message_block, a restatement of Edgewise.forward_node).

Bars: fp32 within 1e-5 of the output scale (max |ref|); bf16 within 2e-2 of
the output scale, the oracle being evaluated in fp64 on the bf16-rounded
inputs, radial scales and weights (the reference path itself is fp32-only).
Segment sums are checked bitwise for run-to-run determinism.
"""
import math

import numpy as np
import pytest
import torch

from oracle import message as omsg
from oracle import rotation as orot

pytestmark = pytest.mark.gpu


def _conv(lmax, mmax, c_in, c_out, gen, gate):
    m_size = [lmax - m + 1 for m in range(mmax + 1)]
    extra = lmax * c_out if gate else 0
    k0 = m_size[0] * c_in
    w0 = torch.randn(m_size[0] * c_out + extra, k0, generator=gen, dtype=torch.float64) / math.sqrt(k0)
    b0 = torch.randn(m_size[0] * c_out + extra, generator=gen, dtype=torch.float64) * 0.1
    wm = []
    for m in range(1, mmax + 1):
        k = m_size[m] * c_in
        wm.append(torch.randn(2 * m_size[m] * c_out, k, generator=gen, dtype=torch.float64) / math.sqrt(k) / math.sqrt(2))
    return {"w0": w0, "b0": b0, "wm": wm, "c_out": c_out}


def _graph(N, E, gen, star=False):
    src = torch.randint(0, N, (E,), generator=gen)
    dst = torch.randint(0, max(1, N - 3), (E,), generator=gen)   # last nodes: no in-edges
    if star:
        dst[: E // 2] = 1                                           # one node with > 64 in-edges
    return torch.stack([src, dst])


def _run(lmax, mmax, dtype, gate, use_rad, N, E, c_in, c_out, seed, device, star=False):
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    gen = torch.Generator().manual_seed(seed)
    d = (lmax + 1) ** 2
    x = torch.randn(N, d, c_in, generator=gen, dtype=torch.float64)
    ei = _graph(N, E, gen, star)
    conv = _conv(lmax, mmax, c_in, c_out, gen, gate)
    kr = M.rad_width(lmax, mmax, c_in)
    rad = (torch.rand(E, kr, generator=gen, dtype=torch.float64) + 0.5) if use_rad else None
    vec = torch.randn(E, 3, generator=gen).float().to(device)
    eul = extract_euler_angles(vec, seed=seed)                      # original edge order
    # quantise inputs the way the device path sees them
    q = (lambda t: t.to(dtype).double()) if dtype == torch.bfloat16 else (lambda t: t.float().double())
    xq, radq = q(x), (q(rad) if rad is not None else None)
    convq = {"w0": q(conv["w0"]), "b0": conv["b0"].float().double(), "wm": [q(w) for w in conv["wm"]],
             "c_out": c_out}
    e64 = eul.cpu().double()
    ref = omsg.message_block(xq, ei, (e64[:, 0], e64[:, 1], e64[:, 2]), orot.load_jd(), lmax, mmax,
                             convq, rad=radq, gate=gate)
    plan = M.MessagePlan(ei.to(device), N)
    outs = []
    for _ in range(2):
        out = M.message_forward(x.to(device=device, dtype=dtype), plan, plan.sort_edges(eul),
                                plan.sort_edges(rad.to(device)) if rad is not None else None,
                                conv["w0"].to(device).float(), conv["b0"].to(device).float(),
                                [w.to(device).float() for w in conv["wm"]], lmax, mmax, gate=gate)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]), "fused block is not run-to-run deterministic"
    got = outs[0].cpu().double()
    scale = ref.abs().max().item()
    err = (got - ref).abs().max().item() / max(scale, 1e-30)
    return err, got, ref


@pytest.mark.parametrize("lmax,mmax", [(2, 2), (4, 2), (6, 2), (4, 4), (6, 6)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("gate", [False, True])
def test_forward_matches_oracle(lmax, mmax, dtype, gate, device):
    print(f"case lmax={lmax} mmax={mmax} dtype={dtype} gate={gate}", flush=True)
    err, got, ref = _run(lmax, mmax, dtype, gate, True, N=40, E=530, c_in=32, c_out=64, seed=lmax * 10 + int(gate),
                         device=device)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert err < tol, f"rel err {err}"
    assert torch.all(got[-3:] == 0), "nodes without in-edges must be exactly zero"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_forward_no_radial_star_graph(dtype, device):
    """A node with > 64 in-edges spans several tiles (partials + fixup)."""
    err, _, _ = _run(4, 2, dtype, False, False, N=20, E=400, c_in=16 if dtype == torch.bfloat16 else 8,
                     c_out=32, seed=3, device=device, star=True)
    assert err < (1e-5 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("lmax,mmax", [(2, 2), (4, 2), (6, 2), (4, 4), (6, 6)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("use_rad", [True, False])
def test_edgewise_two_conv_matches_oracle(lmax, mmax, dtype, use_rad, device):
    """Edgewise with two convolutions on cat(x[src], x[dst]): conv1 gated with
    radial scales, its rows kept in the edge frame (bf16 there for bf16), conv2,
    rotation back and segment sum, against the oracle in fp64."""
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    print(f"edgewise case lmax={lmax} mmax={mmax} dtype={dtype} rad={use_rad}", flush=True)
    N, E, C, H = 33, 470, 32, 64
    gen = torch.Generator().manual_seed(200 + lmax * 3 + int(use_rad))
    d = (lmax + 1) ** 2
    x = torch.randn(N, d, C, generator=gen, dtype=torch.float64)
    ei = _graph(N, E, gen, star=(lmax == 4))
    conv1 = _conv(lmax, mmax, 2 * C, H, gen, True)
    conv2 = _conv(lmax, mmax, H, C, gen, False)
    rad = (torch.rand(E, M.rad_width(lmax, mmax, 2 * C), generator=gen, dtype=torch.float64) + 0.5) \
        if use_rad else None
    eul = extract_euler_angles(torch.randn(E, 3, generator=gen).float().to(device), seed=lmax)
    q = (lambda t: t.to(dtype).double()) if dtype == torch.bfloat16 else (lambda t: t.float().double())
    cq = lambda c: {"w0": q(c["w0"]), "b0": c["b0"].float().double(), "wm": [q(w) for w in c["wm"]],
                    "c_out": c["c_out"]}
    e64 = eul.cpu().double()
    ref = omsg.message_block(q(x), ei, (e64[:, 0], e64[:, 1], e64[:, 2]), orot.load_jd(), lmax, mmax, cq(conv1),
                             rad=q(rad) if rad is not None else None, conv2=cq(conv2), gate=True,
                             concat="source-target")
    plan = M.MessagePlan(ei.to(device), N)
    dv = lambda c: (c["w0"].to(device).float(), c["b0"].to(device).float(), [w.to(device).float() for w in c["wm"]])
    outs = [M.edgewise_forward(x.to(device=device, dtype=dtype), plan, plan.sort_edges(eul),
                               plan.sort_edges(rad.to(device)) if rad is not None else None,
                               dv(conv1), dv(conv2), lmax, mmax) for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]), "not run-to-run deterministic"
    got = outs[0].cpu().double()
    scale = ref.abs().max().item()
    err = (got - ref).abs().max().item() / scale
    assert err < (1e-5 if dtype == torch.float32 else 2e-2), f"rel err {err}"
    assert torch.all(got[-3:] == 0), "nodes without in-edges must be exactly zero"


@pytest.mark.parametrize("lmax,mmax,dtype,mode", [(2, 2, torch.float32, "node"), (4, 2, torch.float32, "node"),
                                                  (6, 2, torch.float32, "node"), (4, 2, torch.float32, "edge"),
                                                  (4, 2, torch.bfloat16, "node"), (2, 2, torch.bfloat16, "edge"),
                                                  (6, 2, torch.bfloat16, "node"), (6, 2, torch.bfloat16, "edge"),
                                                  (4, 4, torch.float32, "node"), (4, 4, torch.bfloat16, "edge"),
                                                  (6, 6, torch.float32, "node"), (6, 6, torch.bfloat16, "node")])
def test_edgewise_gradients_match_oracle_autograd(lmax, mmax, dtype, mode, device):
    """Gradients of the two-convolution block (x, radial scales, both
    convolutions' weights and biases) against fp64 autograd of the oracle."""
    _edgewise_gradient_case(lmax, mmax, dtype, mode, device, C=32, H=64, seed=300 + lmax)


@pytest.mark.parametrize("lmax,mmax", [(4, 2), (6, 2), (4, 4)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_edgewise_gradients_three_channel_blocks(lmax, mmax, dtype, device):
    """96 channels: three 32-channel output blocks per edge tile (an odd count
    in the workgroup -> (tile, channel block) mapping, a 192-channel conv1
    input), every kernel of the block forward and backward; lmax 6 runs the
    8-wave kernels with the gate rows on the light waves."""
    _edgewise_gradient_case(lmax, mmax, dtype, "node", device, C=96, H=96, seed=311 + lmax + mmax)


def _edgewise_gradient_case(lmax, mmax, dtype, mode, device, C, H, seed):
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    print(f"edgewise grad case lmax={lmax} mmax={mmax} dtype={dtype} mode={mode} C={C} H={H}", flush=True)
    N, E = 21, 260
    gen = torch.Generator().manual_seed(seed)
    d = (lmax + 1) ** 2
    x = torch.randn(N, d, C, generator=gen, dtype=torch.float64)
    ei = _graph(N, E, gen, star=(lmax == 4))
    conv1 = _conv(lmax, mmax, 2 * C, H, gen, True)
    conv2 = _conv(lmax, mmax, H, C, gen, False)
    rad = torch.rand(E, M.rad_width(lmax, mmax, 2 * C), generator=gen, dtype=torch.float64) + 0.5
    gout = torch.randn(N if mode == "node" else E, d, C, generator=gen, dtype=torch.float64)
    eul = extract_euler_angles(torch.randn(E, 3, generator=gen).float().to(device), seed=lmax)
    q = (lambda t: t.to(dtype).double()) if dtype == torch.bfloat16 else (lambda t: t.float().double())
    # oracle leaves: the device-visible (quantised) values in fp64
    leaves = [q(x), q(rad), q(conv1["w0"]), conv1["b0"].float().double(), *[q(w) for w in conv1["wm"]],
              q(conv2["w0"]), conv2["b0"].float().double(), *[q(w) for w in conv2["wm"]]]
    leaves = [t.clone().requires_grad_() for t in leaves]
    xo, ro, w01, b01 = leaves[:4]
    wm1 = leaves[4:4 + mmax]
    w02, b02 = leaves[4 + mmax:6 + mmax]
    wm2 = leaves[6 + mmax:]
    e64 = eul.cpu().double()
    ref = omsg.message_block(xo, ei, (e64[:, 0], e64[:, 1], e64[:, 2]), orot.load_jd(), lmax, mmax,
                             {"w0": w01, "b0": b01, "wm": wm1, "c_out": H}, rad=ro,
                             conv2={"w0": w02, "b0": b02, "wm": wm2, "c_out": C}, gate=True,
                             concat="source-target", reduce=(mode == "node"))
    ref.backward(gout)
    plan = M.MessagePlan(ei.to(device), N)
    dl = [t.detach().to(device) for t in leaves]
    dl[0] = dl[0].to(dtype)
    dl = [t.float().requires_grad_() if i > 0 else t.requires_grad_() for i, t in enumerate(dl)]
    rad_d = plan.sort_edges(dl[1].detach()).requires_grad_()
    out = M.edgewise_block(dl[0], plan, plan.sort_edges(eul), rad_d, (dl[2], dl[3], dl[4:4 + mmax]),
                           (dl[4 + mmax], dl[5 + mmax], dl[6 + mmax:]), lmax, mmax, node_or_edge=mode)
    out.backward(gout.to(device).float())
    torch.cuda.synchronize()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    got = {"x": dl[0].grad, "rad": torch.empty_like(rad_d.grad).index_copy_(0, plan.perm, rad_d.grad)}
    names = ["w01", "b01"] + [f"w{m}1" for m in range(1, mmax + 1)] + ["w02", "b02"] + \
        [f"w{m}2" for m in range(1, mmax + 1)]
    got.update({n: t.grad for n, t in zip(names, dl[2:])})
    want = {"x": xo.grad, "rad": ro.grad}
    want.update({n: t.grad for n, t in zip(names, leaves[2:])})
    for n in want:
        scale = want[n].abs().max().item()
        err = (got[n].double().cpu() - want[n]).abs().max().item() / scale
        assert err < tol, (n, err)


@pytest.mark.parametrize("dtype,mode", [(torch.float32, "node"), (torch.bfloat16, "node"), (torch.float32, "edge")])
def test_edgewise_source_target_message(dtype, mode, device):
    """Three-part message cat(x[src], x[dst], x_message_edge): output and every
    gradient (x_message_edge included) against fp64 autograd of the oracle."""
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    print(f"edgewise 3-part case dtype={dtype} mode={mode}", flush=True)
    lmax, mmax, N, E, C, H = 4, 2, 19, 230, 32, 64
    gen = torch.Generator().manual_seed(404)
    d = (lmax + 1) ** 2
    x = torch.randn(N, d, C, generator=gen, dtype=torch.float64)
    xm = torch.randn(E, d, C, generator=gen, dtype=torch.float64)
    ei = _graph(N, E, gen, star=True)
    conv1 = _conv(lmax, mmax, 3 * C, H, gen, True)
    conv2 = _conv(lmax, mmax, H, C, gen, False)
    rad = torch.rand(E, M.rad_width(lmax, mmax, 3 * C), generator=gen, dtype=torch.float64) + 0.5
    gout = torch.randn(N if mode == "node" else E, d, C, generator=gen, dtype=torch.float64)
    eul = extract_euler_angles(torch.randn(E, 3, generator=gen).float().to(device), seed=9)
    q = (lambda t: t.to(dtype).double()) if dtype == torch.bfloat16 else (lambda t: t.float().double())
    leaves = [q(x), q(xm), q(rad), q(conv1["w0"]), conv1["b0"].float().double(), *[q(w) for w in conv1["wm"]],
              q(conv2["w0"]), conv2["b0"].float().double(), *[q(w) for w in conv2["wm"]]]
    leaves = [t.clone().requires_grad_() for t in leaves]
    xo, xmo, ro, w01, b01, w11, w21, w02, b02, w12, w22 = leaves
    e64 = eul.cpu().double()
    ref = omsg.message_block(xo, ei, (e64[:, 0], e64[:, 1], e64[:, 2]), orot.load_jd(), lmax, mmax,
                             {"w0": w01, "b0": b01, "wm": [w11, w21], "c_out": H}, rad=ro,
                             conv2={"w0": w02, "b0": b02, "wm": [w12, w22], "c_out": C}, gate=True,
                             concat="source-target-message", x_message_edge=xmo, reduce=(mode == "node"))
    ref.backward(gout)
    plan = M.MessagePlan(ei.to(device), N)
    dl = [t.detach().to(device) for t in leaves]
    dl[0], dl[1] = dl[0].to(dtype), dl[1].to(dtype)
    dl = [(t if i < 2 else t.float()).requires_grad_() for i, t in enumerate(dl)]
    rad_d = plan.sort_edges(dl[2].detach()).requires_grad_()
    out = M.edgewise_block(dl[0], plan, plan.sort_edges(eul), rad_d, (dl[3], dl[4], dl[5:7]),
                           (dl[7], dl[8], dl[9:11]), lmax, mmax, node_or_edge=mode, x_message_edge=dl[1])
    out.backward(gout.to(device).float())
    torch.cuda.synchronize()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    scale = ref.abs().max().item()
    assert (out.detach().double().cpu() - ref.detach()).abs().max().item() < tol * scale
    got = {"x": dl[0].grad, "xm": dl[1].grad,
           "rad": torch.empty_like(rad_d.grad).index_copy_(0, plan.perm, rad_d.grad)}
    names = ["w01", "b01", "w11", "w21", "w02", "b02", "w12", "w22"]
    got.update({n: t.grad for n, t in zip(names, dl[3:])})
    want = {"x": xo.grad, "xm": xmo.grad, "rad": ro.grad}
    want.update({n: t.grad for n, t in zip(names, leaves[3:])})
    for n in want:
        scale = want[n].abs().max().item()
        err = (got[n].double().cpu() - want[n]).abs().max().item() / scale
        assert err < tol, (n, err)


def test_edgewise_empty_graph(device):
    """No edges: node sums are zero, gradients of x and of every weight are zero."""
    from maloq_amd import message as M
    lmax, mmax, N, C, H = 2, 2, 4, 32, 64
    gen = torch.Generator().manual_seed(1)
    plan = M.MessagePlan(torch.zeros(2, 0, dtype=torch.long, device=device), N)
    c1 = _conv(lmax, mmax, 2 * C, H, gen, True)
    c2 = _conv(lmax, mmax, H, C, gen, False)
    dv = lambda c: (c["w0"].float().to(device).requires_grad_(), c["b0"].float().to(device).requires_grad_(),
                    [w.float().to(device).requires_grad_() for w in c["wm"]])
    conv1, conv2 = dv(c1), dv(c2)
    x = torch.randn(N, 9, C, device=device, requires_grad=True)
    rad = torch.zeros(0, M.rad_width(lmax, mmax, 2 * C), device=device, requires_grad=True)
    out = M.edgewise_block(x, plan, torch.zeros(0, 3, device=device), rad, conv1, conv2, lmax, mmax)
    assert out.shape == (N, 9, C) and torch.all(out == 0)
    out.backward(torch.ones_like(out))
    assert torch.all(x.grad == 0)
    for t in [conv1[0], conv1[1], *conv1[2], conv2[0], conv2[1], *conv2[2]]:
        assert t.grad is not None and torch.all(t.grad == 0)


def test_forward_empty_graph(device):
    from maloq_amd import message as M
    plan = M.MessagePlan(torch.zeros(2, 0, dtype=torch.long, device=device), 5)
    w0 = torch.randn(5 * 32, 5 * 32, device=device)
    wm = [torch.randn(2 * 4 * 32, 4 * 32, device=device), torch.randn(2 * 3 * 32, 3 * 32, device=device)]
    out = M.message_forward(torch.randn(5, 25, 32, device=device), plan, torch.zeros(0, 3, device=device),
                            None, w0, None, wm, 4, 2)
    assert out.shape == (5, 25, 32) and torch.all(out == 0)


def test_config2_scale_against_oracle_subset(device):
    """Config-2 graph (32 x 40 atoms, ~30k edges, lmax 4, C 128) in bf16: the
    nodes of the first molecule against the oracle (their in-edges only)."""
    from maloq_amd import message as M
    from maloq_amd.synth import config2_graph
    from maloq_amd.wigner import extract_euler_angles
    g = config2_graph()
    lmax, mmax, C = 4, 2, 128
    gen = torch.Generator().manual_seed(0)
    N, E = g.num_nodes, g.num_edges
    x = torch.randn(N, 25, C, generator=gen, dtype=torch.float64)
    conv = _conv(lmax, mmax, C, C, gen, False)
    rad = torch.rand(E, M.rad_width(lmax, mmax, C), generator=gen, dtype=torch.float64) + 0.5
    ei = torch.from_numpy(np.stack([g.src, g.dst]))
    vec = torch.from_numpy(g.edge_distance_vec()).float().to(device)
    eul = extract_euler_angles(vec, seed=1)
    plan = M.MessagePlan(ei.to(device), N)
    dt = torch.bfloat16
    out = M.message_forward(x.to(device=device, dtype=dt), plan, plan.sort_edges(eul),
                            plan.sort_edges(rad.to(device)), conv["w0"].to(device).float(),
                            conv["b0"].to(device).float(), [w.to(device).float() for w in conv["wm"]],
                            lmax, mmax)
    mol0 = np.nonzero(g.mol == 0)[0]
    sel = np.isin(g.dst, mol0)
    q = lambda t: t.to(dt).double()
    e64 = eul.cpu().double()[torch.from_numpy(sel)]
    ref = omsg.message_block(q(x), ei[:, torch.from_numpy(sel)], (e64[:, 0], e64[:, 1], e64[:, 2]),
                             orot.load_jd(), lmax, mmax,
                             {"w0": q(conv["w0"]), "b0": conv["b0"].float().double(),
                              "wm": [q(w) for w in conv["wm"]], "c_out": C},
                             rad=q(rad)[torch.from_numpy(sel)])
    got = out.cpu().double()[mol0]
    err = (got - ref[mol0]).abs().max().item() / ref[mol0].abs().max().item()
    assert err < 2e-2, err


@pytest.mark.parametrize("lmax,mmax", [(2, 2), (4, 2), (6, 2), (4, 4), (6, 6)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("gate", [False, True])
def test_backward_matches_oracle_autograd(lmax, mmax, dtype, gate, device):
    """Gradients of x, rad, W0, b0 and W_m against fp64 autograd through the
    oracle; gated blocks (GateActivation, activation.py:57-77) included."""
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    print(f"bwd case lmax={lmax} dtype={dtype} gate={gate}", flush=True)
    gen = torch.Generator().manual_seed(100 + lmax + 7 * int(gate))
    N, E, c_in, c_out = 30, 300, 32, 32
    d = (lmax + 1) ** 2
    q = (lambda t: t.to(dtype).double()) if dtype == torch.bfloat16 else (lambda t: t.float().double())
    x = q(torch.randn(N, d, c_in, generator=gen, dtype=torch.float64))
    ei = _graph(N, E, gen)
    conv = _conv(lmax, mmax, c_in, c_out, gen, gate)
    conv = {"w0": q(conv["w0"]), "b0": conv["b0"].float().double(), "wm": [q(w) for w in conv["wm"]], "c_out": c_out}
    rad = q(torch.rand(E, M.rad_width(lmax, mmax, c_in), generator=gen, dtype=torch.float64) + 0.5)
    gout = torch.randn(N, d, c_out, generator=gen, dtype=torch.float64)
    vec = torch.randn(E, 3, generator=gen).float().to(device)
    eul = extract_euler_angles(vec, seed=7)
    e64 = eul.cpu().double()
    leaves = [x.clone().requires_grad_(), rad.clone().requires_grad_(), conv["w0"].clone().requires_grad_(),
              conv["b0"].clone().requires_grad_()] + [w.clone().requires_grad_() for w in conv["wm"]]
    ref = omsg.message_block(leaves[0], ei, (e64[:, 0], e64[:, 1], e64[:, 2]), orot.load_jd(), lmax, mmax,
                             {"w0": leaves[2], "b0": leaves[3], "wm": leaves[4:], "c_out": c_out}, rad=leaves[1],
                             gate=gate)
    (ref * gout).sum().backward()
    plan = M.MessagePlan(ei.to(device), N)
    dl = [x.to(device=device, dtype=dtype).requires_grad_(),
          plan.sort_edges(rad.to(device=device, dtype=dtype)).requires_grad_(),
          conv["w0"].to(device).float().requires_grad_(), conv["b0"].to(device).float().requires_grad_()] + \
         [w.to(device).float().requires_grad_() for w in conv["wm"]]
    out = M.message_block(dl[0], plan, plan.sort_edges(eul), dl[1], dl[2], dl[3], dl[4:], lmax, mmax, gate=gate)
    out.backward(gout.float().to(device))
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    inv = torch.empty_like(plan.perm)
    inv[plan.perm] = torch.arange(E, device=device)
    names = ["x", "rad", "w0", "b0"] + [f"w{m}" for m in range(1, mmax + 1)]
    for name, a, b in zip(names, dl, leaves):
        ga = a.grad
        if name == "rad":
            ga = ga[inv]   # back to the original edge order
        ga = ga.cpu().double()
        err = (ga - b.grad).abs().max().item() / max(b.grad.abs().max().item(), 1e-30)
        assert err < tol, f"grad {name}: rel err {err}"


# first run together with a GPU build that faulted the GPU (32-edge forward tiles at three workgroups
# per CU); the faulting case is not identified, so these never-before-run shapes stay off the GPU
_SKIP_C256 = pytest.mark.skip(reason="first run in a GPU run that faulted; faulting case not identified")


@pytest.mark.parametrize("lmax,mmax,c_in,c_out,E,splits", [(4, 2, 128, 128, 1000, None), (4, 2, 128, 128, 1000, 3),
                                                          (2, 2, 32, 64, 37, None), (6, 2, 64, 32, 260, 2),
                                                          (4, 4, 128, 64, 517, None), (6, 6, 32, 32, 300, 2),
                                                          pytest.param(4, 2, 256, 256, 1000, None, marks=_SKIP_C256),
                                                          pytest.param(4, 2, 256, 256, 701, 2, marks=_SKIP_C256)])
def test_weight_grad_bf16_against_fp64(lmax, mmax, c_in, c_out, E, splits, device):
    """maloq_message_dw (bf16): ragged edge counts, partial 256-column tiles,
    several split-K ranges; against fp64 sums of the same bf16 rows, with the
    +-m folding of so2_layers.py:61-67 (dWr = C++ + C--, dWi = C-+ - C+-)."""
    from maloq_amd import message as M
    print(f"dw case lmax={lmax} mmax={mmax} c_in={c_in} c_out={c_out} E={E} splits={splits}", flush=True)
    gen = torch.Generator().manual_seed(E + lmax)
    P = M.kept_rows(lmax, mmax)
    dz = M._edge_rows(E, P, c_out, device, torch.bfloat16)
    y = M._edge_rows(E, P, c_in, device, torch.bfloat16)
    dz[:E] = torch.randn(E, P, c_out, generator=gen).to(device=device, dtype=torch.bfloat16)
    y[:E] = torch.randn(E, P, c_in, generator=gen).to(device=device, dtype=torch.bfloat16)
    dw0, dwm, db0 = M.message_weight_grad(dz, y, lmax, mmax, c_out, c_in, splits=splits, num_edges=E)
    torch.cuda.synchronize()
    dzd, yd = dz[:E].double().cpu(), y[:E].double().cpu()
    r0 = lmax + 1
    ref0 = torch.einsum("en,ek->nk", dzd[:, :r0].reshape(E, -1), yd[:, :r0].reshape(E, -1))
    scale = ref0.abs().max().item()
    assert (dw0.double().cpu() - ref0).abs().max().item() / scale < 1e-5
    row = r0
    for m in range(1, mmax + 1):
        nr = lmax - m + 1
        Cm = torch.einsum("en,ek->nk", dzd[:, row:row + 2 * nr].reshape(E, -1), yd[:, row:row + 2 * nr].reshape(E, -1))
        ho, hi = nr * c_out, nr * c_in
        dwr = Cm[:ho, :hi] + Cm[ho:, hi:]
        dwi = Cm[ho:, :hi] - Cm[:ho, hi:]
        ref = torch.cat([dwr, dwi])
        err = (dwm[m - 1].double().cpu() - ref).abs().max().item() / ref.abs().max().item()
        assert err < 1e-5, (m, err)
        row += 2 * nr
    assert torch.allclose(db0.double().cpu(), dzd[:, :r0].sum(0).reshape(-1), rtol=1e-5, atol=1e-3)
