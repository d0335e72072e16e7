"""Fock_Irreps_Head on the GPU (maloq_amd.irreps_head; reference
helm/esen_osh.py:522-1064) against the fp64 CPU restatement: labels and every
gradient (node and edge embeddings, all parameters), plain, reduce_node (with
and without reduce_node_intra) and reduce_edge, closed and open shell."""
import numpy as np
import pytest
import torch

from maloq_amd import tensor_decomp as ptd
from oracle import irreps_head as oh

pytestmark = pytest.mark.gpu

CFG3 = {1: [0, 0, 1], 6: [0, 0, 0, 1, 1, 2], 7: [0, 0, 0, 1, 1, 2], 8: [0, 0, 0, 1, 1, 2]}


def _oracle_params(mod, spins):
    d = lambda t: t.detach().double().cpu()
    out = []
    for s in range(spins):
        ls = mod.lin_scalars_learnable[s]
        p = {"scalar": (d(ls.weight), d(ls.bias))}
        streams = ({"node": mod.node_lin_out_layers, "edge": mod.edge_lin_out_layers} if mod.reduce_node
                   else {"common": mod.lin_out_layers})
        for name, layers in streams.items():
            p[name] = ([d(lin.weight) for lin in layers[s]], d(layers[s][0].bias))
        out.append(p)
    return out


@pytest.mark.parametrize("reduce_node,intra,open_shell", [(False, False, False), (True, True, False),
                                                          (True, False, False), (True, True, True)])
def test_head_matches_oracle(reduce_node, intra, open_shell):
    from maloq_amd.irreps_head import Fock_Irreps_Head
    t = ptd.BasisTables({k: list(v) for k, v in CFG3.items()})
    ls_list = t.ls_list
    irreps_out = t.req_output_irreps
    lmax, C = max(oh.all_ls(ls_list)), 32
    irreps_in = "+".join(f"{C}x{l}e" for l in range(lmax + 1))
    torch.manual_seed(5)
    mod = Fock_Irreps_Head(irreps_in, irreps_out, lmax, C, ls_list=ls_list, reduce_node=reduce_node,
                           reduce_node_intra=intra, open_shell=open_shell).cuda()
    with torch.no_grad():   # non-zero biases, so their paths are exercised
        for name, p in mod.named_parameters():
            if name.endswith("bias") and p.numel():
                p.copy_(0.3 * torch.randn_like(p))
    gen = torch.Generator().manual_seed(1)
    d = (lmax + 1) ** 2
    xn = torch.randn(37, d, C, generator=gen)
    xe = torch.randn(211, d, C, generator=gen)
    xn_d, xe_d = xn.cuda().requires_grad_(), xe.cuda().requires_grad_()
    node, edge = mod({"node_embeddings": xn_d, "edge_embeddings": xe_d}, None)
    spins = 2 if open_shell else 1
    T = sum(2 * l + 1 for l in oh.all_ls(ls_list))
    assert node.shape == (spins, 37, T) and edge.shape == (spins, 211, T)
    gn = torch.randn(node.shape, generator=gen)
    ge = torch.randn(edge.shape, generator=gen)
    (node * gn.cuda()).sum().add((edge * ge.cuda()).sum()).backward()

    params = _oracle_params(mod, spins)
    leaves = [xn.double().requires_grad_(), xe.double().requires_grad_()]
    flat = []
    for p in params:
        for v in p.values():
            for t_ in (v[0] if isinstance(v[0], list) else [v[0]]) + [v[1]]:
                t_.requires_grad_()
                flat.append(t_)
    n_ref, e_ref = oh.head_forward(leaves[0], leaves[1], ls_list, lmax, C, params, reduce_node, intra, spins)
    (n_ref * gn.double()).sum().add((e_ref * ge.double()).sum()).backward()

    def close(got, ref, what):
        got = got.detach().double().cpu()
        err = (got - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
        assert err < 1e-5, f"{what}: rel err {err:.2e}"

    close(node, n_ref.detach(), "node labels")
    close(edge, e_ref.detach(), "edge labels")
    close(xn_d.grad, leaves[0].grad, "grad node embeddings")
    close(xe_d.grad, leaves[1].grad, "grad edge embeddings")
    # parameters, in the order _oracle_params visits them
    mods = []
    for s in range(spins):
        mods.append(mod.lin_scalars_learnable[s])
        streams = ([mod.node_lin_out_layers, mod.edge_lin_out_layers] if reduce_node else [mod.lin_out_layers])
        for layers in streams:
            mods.append(("layers", layers[s]))
    k = 0
    for m in mods:
        if isinstance(m, tuple):
            for lin in m[1]:
                if lin.weight.numel():
                    close(lin.weight.grad, flat[k].grad, f"grad {lin.l} weight")
                k += 1
            if m[1][0].bias.numel():
                close(m[1][0].bias.grad, flat[k].grad, "grad l0 bias")
            k += 1
        else:
            close(m.weight.grad, flat[k].grad, "grad scalar weight")
            close(m.bias.grad, flat[k + 1].grad, "grad scalar bias")
            k += 2


def test_state_dict_names_follow_the_reference():
    from maloq_amd.irreps_head import Fock_Irreps_Head
    t = ptd.BasisTables({k: list(v) for k, v in CFG3.items()})
    mod = Fock_Irreps_Head("+".join(f"16x{l}e" for l in range(5)), t.req_output_irreps, 4, 16, ls_list=t.ls_list,
                           reduce_node=True, reduce_node_intra=True)
    keys = set(mod.state_dict())
    for k in ("lin_scalars_learnable.0.weight", "lin_scalars_learnable.0.bias", "node_lin_out_layers.0.0.weight",
              "node_lin_out_layers.0.0.bias", "edge_lin_out_layers.0.4.weight"):
        assert k in keys, k
    with pytest.raises(NotImplementedError):   # reduce_edge without reduce_node (esen_osh.py:597-598)
        Fock_Irreps_Head("16x0e", t.req_output_irreps, 4, 16, ls_list=t.ls_list, reduce_edge=True)
    red = Fock_Irreps_Head("+".join(f"16x{l}e" for l in range(5)), t.req_output_irreps, 4, 16, ls_list=t.ls_list,
                           reduce_node=True, reduce_node_intra=True, reduce_edge=True)
    keys = set(red.state_dict())
    for k in ("edge_lin_out_layers.alpha.0.4.weight", "edge_lin_out_layers.beta.0.1.weight",
              "node_lin_out_layers.0.0.bias", "lin_scalars_learnable.0.weight"):
        assert k in keys, k


def _pair_graph(n_nodes, n_pairs, seed):
    """edge_index with every edge and its reverse, in shuffled order."""
    rng = np.random.default_rng(seed)
    pairs = set()
    while len(pairs) < n_pairs:
        i, j = rng.integers(0, n_nodes, 2)
        if i != j:
            pairs.add((min(i, j), max(i, j)))
    e = np.array([p for p in pairs] + [(j, i) for i, j in pairs]).T
    return torch.as_tensor(e[:, rng.permutation(e.shape[1])], dtype=torch.int64)


@pytest.mark.parametrize("open_shell", [False, True])
def test_reduce_edge_head_matches_oracle(open_shell):
    from maloq_amd.irreps_head import Fock_Irreps_Head
    t = ptd.BasisTables({k: list(v) for k, v in CFG3.items()})
    ls_list = t.ls_list
    lmax, C = max(oh.all_ls(ls_list)), 32
    irreps_in = "+".join(f"{C}x{l}e" for l in range(lmax + 1))
    torch.manual_seed(7)
    mod = Fock_Irreps_Head(irreps_in, t.req_output_irreps, lmax, C, ls_list=ls_list, reduce_node=True,
                           reduce_node_intra=True, reduce_edge=True, open_shell=open_shell).cuda()
    with torch.no_grad():
        for name, p in mod.named_parameters():
            if name.endswith("bias") and p.numel():
                p.copy_(0.3 * torch.randn_like(p))
    names = dict(mod.named_parameters())
    assert all(names[f"edge_lin_out_layers.{s}.0.0.bias"].numel() == 0 for s in ("alpha", "beta"))
    assert names["lin_scalars_learnable.0.bias"].numel() == 0
    ei = _pair_graph(37, 150, 2)
    E = ei.shape[1]
    gen = torch.Generator().manual_seed(3)
    d = (lmax + 1) ** 2
    xn = torch.randn(37, d, C, generator=gen)
    xe = torch.randn(E, d, C, generator=gen)
    xn_d, xe_d = xn.cuda().requires_grad_(), xe.cuda().requires_grad_()
    node, edge = mod({"node_embeddings": xn_d, "edge_embeddings": xe_d}, {"edge_index": ei.cuda()})
    spins = 2 if open_shell else 1
    T = sum(2 * l + 1 for l in oh.all_ls(ls_list))
    assert node.shape == (spins, 37, T) and edge.shape == (spins, E, T)
    gn, ge = torch.randn(node.shape, generator=gen), torch.randn(edge.shape, generator=gen)
    (node * gn.cuda()).sum().add((edge * ge.cuda()).sum()).backward()

    ref = {n: p.detach().double().cpu().requires_grad_() for n, p in names.items()}
    nl = lambda k, s: [ref[f"{k}.{s}.{l}.weight"] for l in range(lmax + 1)]
    params = [{"scalar": (ref[f"lin_scalars_learnable.{s}.weight"], None),
               "node": (nl("node_lin_out_layers", s), ref[f"node_lin_out_layers.{s}.0.bias"]),
               "alpha": (nl(f"edge_lin_out_layers.alpha", s), None),
               "beta": (nl(f"edge_lin_out_layers.beta", s), None)} for s in range(spins)]
    xn64, xe64 = xn.double().requires_grad_(), xe.double().requires_grad_()
    n_ref, e_ref = oh.head_forward(xn64, xe64, ls_list, lmax, C, params, True, True, spins, reduce_edge=True,
                                   edge_index=ei)
    (n_ref * gn.double()).sum().add((e_ref * ge.double()).sum()).backward()

    def close(got, want, what):
        got = got.detach().double().cpu()
        err = (got - want).abs().max().item() / max(want.abs().max().item(), 1e-30)
        assert err < 1e-5, f"{what}: rel err {err:.2e}"

    close(node, n_ref.detach(), "node labels")
    close(edge, e_ref.detach(), "edge labels")
    close(xn_d.grad, xn64.grad, "grad node embeddings")
    close(xe_d.grad, xe64.grad, "grad edge embeddings")
    for n, p in names.items():
        if p.numel() and ref[n].grad is not None:
            close(p.grad, ref[n].grad, f"grad {n}")


def test_reduce_edge_needs_reverse_edges():
    from maloq_amd.irreps_head import Fock_Irreps_Head
    t = ptd.BasisTables({k: list(v) for k, v in CFG3.items()})
    lmax, C = max(oh.all_ls(t.ls_list)), 16
    mod = Fock_Irreps_Head("+".join(f"{C}x{l}e" for l in range(lmax + 1)), t.req_output_irreps, lmax, C,
                           ls_list=t.ls_list, reduce_node=True, reduce_node_intra=True, reduce_edge=True).cuda()
    ei = torch.tensor([[0, 1, 1], [1, 0, 2]]).cuda()
    x = torch.randn(3, (lmax + 1) ** 2, C).cuda()
    with pytest.raises(ValueError):
        mod({"node_embeddings": x, "edge_embeddings": torch.randn(3, (lmax + 1) ** 2, C).cuda()}, {"edge_index": ei})
    # no edges at all: empty edge labels, node labels as usual
    T = sum(2 * l + 1 for l in oh.all_ls(t.ls_list))
    n, e = mod({"node_embeddings": x, "edge_embeddings": torch.zeros(0, (lmax + 1) ** 2, C).cuda()},
               {"edge_index": torch.zeros(2, 0, dtype=torch.int64).cuda()})
    assert n.shape == (1, 3, T) and e.shape == (1, 0, T)
