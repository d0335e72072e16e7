"""A whole training step of the fused block, and a forward + backward call of
the drop-in Edgewise module, captured once into a HIP graph (torch.cuda.graph
over the maloq_hip operators) and replayed: the path for launch-bound small
graphs such as config 1, where the host's enqueue of the step's kernels costs
more than the kernels.  The step is the one the benchmark times: Euler
angles, the fused RadialMLP, the block forward and backward.  Every replay,
with eager work between replays, must give the eager call's output and
gradients bit for bit (the kernels are deterministic)."""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _workload(dt, device):
    from maloq_amd import message as M
    from maloq_amd.radial import RadialMLP
    from maloq_amd.synth import config1_graph
    g = config1_graph()
    L = Mm = 2
    C = 32
    gen = torch.Generator().manual_seed(0)
    plan = M.MessagePlan(torch.from_numpy(np.stack([g.src, g.dst])).to(device), g.num_nodes)
    vec = plan.sort_edges(torch.from_numpy(g.edge_distance_vec()).float().to(device))
    offsets = torch.linspace(0.0, 5.0, 8, device=device)
    coeff = -0.5 / float(offsets[1] - offsets[0]) ** 2
    rbf = torch.exp(coeff * (vec.norm(dim=1, keepdim=True) - offsets) ** 2)
    x = torch.randn(g.num_nodes, (L + 1) ** 2, C, generator=gen).to(device=device, dtype=dt).requires_grad_()
    w0 = (torch.randn((L + 1) * C, (L + 1) * C, generator=gen) / math.sqrt((L + 1) * C)).to(device).requires_grad_()
    b0 = torch.zeros((L + 1) * C, device=device, requires_grad=True)
    wm = [(torch.randn(2 * (L - m + 1) * C, (L - m + 1) * C, generator=gen) / math.sqrt((L - m + 1) * C))
          .to(device).requires_grad_() for m in (1, 2)]
    torch.manual_seed(0)
    radial = RadialMLP([8, 64, 64, M.rad_width(L, Mm, C)]).to(device)
    gout = torch.randn(g.num_nodes, (L + 1) ** 2, C, generator=gen).to(device)
    params = [x, w0, b0, *wm, *radial.parameters()]
    return dict(plan=plan, vec=vec, rbf=rbf, x=x, w0=w0, b0=b0, wm=wm, radial=radial, gout=gout, dt=dt,
                L=L, M=Mm, params=params)


def _step(w):
    from maloq_amd import ops
    from maloq_amd.wigner import extract_euler_angles
    eul = extract_euler_angles(w["vec"], seed=1234)
    rad = w["radial"](w["rbf"], out_dtype=w["dt"])
    out = ops.message_block(w["x"], w["plan"], eul, rad, w["w0"], w["b0"], w["wm"], w["L"], w["M"])
    for t in w["params"]:
        t.grad = None
    out.backward(w["gout"])
    return out


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_training_step_replays_from_a_hip_graph(dt, device):
    print(f"graph capture case dtype={dt}", flush=True)
    w = _workload(dt, device)
    _check_replays(lambda: _step(w), w["params"])


def _check_replays(call, leaves):
    """Warm-up (the per-device tables are uploaded here, not during capture),
    capture of one call, the eager reference, and three replays with eager
    work between them, all on one side stream (autograd's gradient
    accumulators then stay on the stream they were made on)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out_g = call()
        grads_g = [t.grad for t in leaves]
        assert all(gr is not None for gr in grads_g)
        # the eager call (new gradient tensors; the graph keeps its own)
        ref = call().detach().clone()
        ref_grads = [t.grad.detach().clone() for t in leaves]
        torch.cuda.synchronize()
        for rep in range(3):
            call()
            (leaves[0].detach().float() * 2).sum()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_g, ref), f"replay {rep}: output differs from the eager call"
            for i, (a, b) in enumerate(zip(grads_g, ref_grads)):
                assert torch.equal(a, b), f"replay {rep}: gradient {i} differs from the eager call"
    torch.cuda.current_stream().wait_stream(s)


@pytest.mark.parametrize("lmax,mmax,C,H,ecl,dense", [
    (4, 2, 32, 64, (8, 32, 32), False),
    # the reference's example layer: lmax = mmax = 4, C = H = 128, radial
    # [384, 128, 128] (torch layers ahead of the fused tail), dense wigner
    (4, 4, 128, 128, (384, 128, 128), True)])
def test_edgewise_layer_replays_from_a_hip_graph(lmax, mmax, C, H, ecl, dense, device):
    """The drop-in Edgewise module, called as the reference's backbone calls
    it (no plan=: the cached plan of the first call), forward and backward
    captured into one HIP graph; every replay bitwise equal to the eager call."""
    from maloq_amd.edgewise import Edgewise
    from maloq_amd.so3 import CoefficientMapping
    from maloq_amd.wigner import extract_euler_angles, wigner_from_eulers
    print(f"graph capture Edgewise case lmax={lmax} mmax={mmax} C={C} dense={dense}", flush=True)
    torch.manual_seed(0)
    mod = Edgewise(C, H, lmax, mmax, list(ecl), CoefficientMapping(lmax, mmax), None, 6.0,
                   "source-target").to(device)
    gen = torch.Generator().manual_seed(7)
    N, E = 23, 300
    x = torch.randn(N, (lmax + 1) ** 2, C, generator=gen).to(device).requires_grad_()
    ei = torch.stack([torch.randint(0, N, (E,), generator=gen), torch.randint(0, N - 2, (E,), generator=gen)])
    ei = ei.to(device)
    x_edge = torch.randn(E, ecl[0], generator=gen).to(device).requires_grad_()
    eul = extract_euler_angles(torch.randn(E, 3, generator=gen).to(device), seed=5)
    w = wigner_from_eulers(eul, None, lmax) if dense else None
    winv = w.transpose(1, 2).contiguous() if dense else None
    gout = torch.randn(N, (lmax + 1) ** 2, C, generator=gen).to(device)
    leaves = [x, x_edge, *mod.parameters()]

    def call():
        out = mod(x, None, x_edge, ei, w, winv, "node", eulers=None if dense else eul)
        for t in leaves:
            t.grad = None
        out.backward(gout)
        return out

    _check_replays(call, leaves)
