"""The energy and force heads' message pass (maloq_amd.heads, the reference's
HELM_Energy_Head / HELM_Force_Head, esen_osh.py:1137-1342) against the oracle:
the two-convolution message block in fp64 (oracle.message with conv2 and
concat "source-target"), its l = 0 row through the module's own MLP and summed
per molecule, or its l = 1 rows; outputs and the gradients of the node
embeddings, the edge features and every parameter within 1e-5 (fp32)."""
import types

import numpy as np
import pytest
import torch

from oracle import message as omsg
from oracle import rotation as orot
from oracle.so2 import radial_mlp

pytestmark = pytest.mark.gpu


def _oracle_rad(mod, params, x_edge64):
    rf = "so2_conv_1.rad_func.net."
    net = mod.so2_conv_1.rad_func.net
    lin = [i for i, m in enumerate(net) if isinstance(m, torch.nn.Linear)]
    lns = [i for i, m in enumerate(net) if isinstance(m, torch.nn.LayerNorm)]
    hidden = [(params[f"{rf}{a}.weight"], params[f"{rf}{a}.bias"], params[f"{rf}{b}.weight"], params[f"{rf}{b}.bias"])
              for a, b in zip(lin[:-1], lns)]
    return radial_mlp(x_edge64, hidden, params[f"{rf}{lin[-1]}.weight"], params[f"{rf}{lin[-1]}.bias"], net[lns[0]].eps)


@pytest.mark.parametrize("kind,lmax,mmax,dense", [("energy", 2, 2, True), ("force", 2, 2, False),
                                                  ("energy", 4, 2, False), ("force", 4, 4, True)])
def test_head_matches_oracle(kind, lmax, mmax, dense, device):
    from maloq_amd import heads
    from maloq_amd.synth import batch_of_molecules
    from maloq_amd.wigner import extract_euler_angles, wigner_from_eulers
    print(f"head case {kind} lmax={lmax} mmax={mmax} dense={dense}", flush=True)
    C = H = 32
    bb = types.SimpleNamespace(sphere_channels=C, hidden_channels=H, lmax=lmax, mmax=mmax,
                               edge_channels_list=[8, 32, 32])
    torch.manual_seed(0)
    mod = (heads.HELM_Energy_Head(bb) if kind == "energy" else heads.HELM_Force_Head(bb)).to(device)
    g = batch_of_molecules(3, lambda m: 7 + 2 * m, ["H", "C", "O"], [0.5, 0.3, 0.2], 5.0)
    gen = torch.Generator().manual_seed(1)
    N, E, d = g.num_nodes, g.num_edges, (lmax + 1) ** 2
    x = torch.randn(N, d, C, generator=gen)
    x_edge = torch.randn(E, 8, generator=gen)
    ei = torch.from_numpy(np.stack([g.src, g.dst]))
    eul = extract_euler_angles(torch.from_numpy(g.edge_distance_vec()).float().to(device), seed=2)
    xd, xed = x.to(device).requires_grad_(), x_edge.to(device).requires_grad_()
    emb = {"node_embeddings": xd, "x_edge": xed}
    if dense:
        w = wigner_from_eulers(eul, None, lmax)
        emb.update(wigner=w, wigner_inv=w.transpose(1, 2))
        kw = {}
    else:
        kw = {"eulers": eul}
    counts = [int(np.sum(g.mol == m)) for m in range(3)]
    batch = types.SimpleNamespace(edge_index=ei.to(device)[None], num_atoms_in_molecule=torch.tensor(counts))
    res = mod(emb, batch, **kw)
    got = res["energies" if kind == "energy" else "forces"]
    gout = torch.randn(got.shape, generator=gen, dtype=torch.float64)
    got.backward(gout.float().to(device))
    # oracle
    params = {k: v.detach().double().cpu().requires_grad_() for k, v in mod.named_parameters()}
    x64, xe64 = x.double().requires_grad_(), x_edge.double().requires_grad_()
    rad = _oracle_rad(mod, params, xe64)
    conv = lambda p, c: {"w0": params[f"{p}.fc_m0.weight"], "b0": params[f"{p}.fc_m0.bias"],
                         "wm": [params[f"{p}.so2_m_conv.{i}.fc.weight"] for i in range(mmax)], "c_out": c}
    e64 = eul.double().cpu()
    new = omsg.message_block(x64, ei, (e64[:, 0], e64[:, 1], e64[:, 2]), orot.load_jd(), lmax, mmax,
                             conv("so2_conv_1", H), rad=rad, conv2=conv("so2_conv_2", mod.out_channels), gate=True,
                             concat="source-target")
    if kind == "energy":
        h = torch.nn.functional.linear(new[:, 0], params["linear.0.weight"], params["linear.0.bias"])
        h = torch.nn.functional.linear(torch.nn.functional.silu(h), params["linear.2.weight"], params["linear.2.bias"])
        per_atom = h[:, 0]
        ref = torch.stack([s.sum() for s in torch.split(per_atom, counts)])
    else:
        ref = new[:, 1:4, 0]
    ref.backward(gout)
    pairs = [("out", got.detach(), ref.detach()), ("x", xd.grad, x64.grad), ("x_edge", xed.grad, xe64.grad)]
    pairs += [(k, v.grad, params[k].grad) for k, v in mod.named_parameters()]
    for name, a, b in pairs:
        scale = b.abs().max().item()
        assert a is not None, name
        assert (a.double().cpu() - b).abs().max().item() <= 1e-5 * max(scale, 1e-30), name
