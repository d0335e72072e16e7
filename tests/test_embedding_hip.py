"""GPU parity of the edge-degree embedding (maloq_edge_degree_embed) against
the CPU oracle (oracle.embedding, a restatement of embedding.py:82-141).

Bars: fp32 within 1e-5 of the output scale, the oracle in fp64 on the same
Euler angles; bf16 within 2e-2 (the oracle on the bf16-rounded radial rows).
The Euler-angle source must give bit-identical results to the dense
wigner_inv source (same recurrence); node sums are checked bitwise for
run-to-run determinism and for nodes without in-edges."""
import pytest
import torch

from oracle import embedding as oemb
from oracle import rotation as orot
from oracle.so3 import CoefficientMapping

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def device():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _case(lmax, N, E, C, seed, device, udt=torch.float32):
    from maloq_amd.wigner import extract_euler_angles, wigner_from_eulers
    gen = torch.Generator().manual_seed(seed)
    vec = torch.randn(E, 3, generator=gen)
    src = torch.randint(0, N, (E,), generator=gen)
    dst = torch.randint(0, max(1, N - 2), (E,), generator=gen)   # last nodes: no in-edges
    ei = torch.stack([src, dst])
    u = torch.randn(E, (lmax + 1) * C, generator=gen).to(udt)
    eul = extract_euler_angles(vec.to(device), seed=seed + 11)
    winv = wigner_from_eulers(eul, orot.load_jd(torch.float32), lmax, inverse=True)
    # oracle D from the same angles in fp64
    e64 = eul.double().cpu()
    w64 = orot.eulers_to_wigner((e64[:, 0], e64[:, 1], e64[:, 2]), 0, lmax, orot.load_jd(torch.float64))
    return ei, u, eul, winv, w64.transpose(1, 2).contiguous()


def _oracle(x, u, ei, winv64, lmax, mode):
    mapping = CoefficientMapping(lmax, 2)
    mask = CoefficientMapping(lmax, lmax).coefficient_idx(lmax, 2)
    return oemb.edge_degree_embedding(x.double(), u.double(), ei, winv64, mapping, mask, 5.0, mode)


@pytest.mark.parametrize("lmax,C", [(2, 16), (4, 128), (6, 64), (4, 256)])
@pytest.mark.parametrize("source", ["wigner_inv", "eulers"])
def test_node_mode_matches_oracle(lmax, C, source, device):
    from maloq_amd.embedding import edge_degree_embed
    print(f"embed node case lmax={lmax} C={C} source={source}", flush=True)
    N, E = 37, 400
    ei, u, eul, winv, w64 = _case(lmax, N, E, C, lmax * 7 + C, device)
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(N, (lmax + 1) ** 2, C, generator=gen)
    kw = {"eulers": eul} if source == "eulers" else {}
    xd = x.to(device)
    with torch.no_grad():
        got = edge_degree_embed(xd, u.to(device), ei.to(device), winv if source == "wigner_inv" else None, lmax, 5.0,
                                "node", **kw)
    assert got.data_ptr() == xd.data_ptr()   # in place, as x.index_add_
    ref = _oracle(x, u, ei, w64, lmax, "node")
    scale = ref.abs().max().item()
    err = (got.double().cpu() - ref).abs().max().item()
    assert err <= 1e-5 * scale, (err, scale)
    assert torch.equal(got[N - 1].cpu(), x[N - 1])     # no in-edges: untouched
    # run-to-run determinism
    with torch.no_grad():
        again = edge_degree_embed(x.to(device), u.to(device), ei.to(device),
                                  winv if source == "wigner_inv" else None, lmax, 5.0, "node", **kw)
    assert torch.equal(got, again)


@pytest.mark.parametrize("lmax", [2, 4, 6])
def test_edge_mode_and_sources_agree(lmax, device):
    from maloq_amd.embedding import edge_degree_embed
    print(f"embed edge case lmax={lmax}", flush=True)
    N, E, C = 20, 333, 32
    ei, u, eul, winv, w64 = _case(lmax, N, E, C, 50 + lmax, device)
    x = torch.zeros(N, (lmax + 1) ** 2, C, device=device)
    ud = u.to(device)
    a = edge_degree_embed(x, ud, ei.to(device), winv, lmax, 5.0, "edge")
    b = edge_degree_embed(x, ud, ei.to(device), None, lmax, 5.0, "edge", eulers=eul)
    assert torch.equal(a, b)
    ref = _oracle(x.cpu(), u, ei, w64, lmax, "edge")
    scale = ref.abs().max().item()
    assert (a.double().cpu() - ref).abs().max().item() <= 1e-5 * scale


def test_bf16_rows_and_nodes(device):
    from maloq_amd.embedding import edge_degree_embed
    lmax, N, E, C = 4, 30, 500, 128
    ei, u, eul, winv, w64 = _case(lmax, N, E, C, 77, device, udt=torch.bfloat16)
    x = torch.zeros(N, (lmax + 1) ** 2, C, dtype=torch.bfloat16)
    with torch.no_grad():
        got = edge_degree_embed(x.to(device), u.to(device), ei.to(device), None, lmax, 5.0, "node", eulers=eul)
    ref = _oracle(x, u, ei, w64, lmax, "node")
    scale = ref.abs().max().item()
    assert (got.double().cpu() - ref).abs().max().item() <= 2e-2 * scale


def test_empty_graph(device):
    from maloq_amd.embedding import edge_degree_embed
    x = torch.randn(4, 25, 8, device=device)
    x0 = x.clone()
    with torch.no_grad():
        out = edge_degree_embed(x, torch.zeros(0, 40, device=device), torch.zeros(2, 0, dtype=torch.long,
                                device=device), None, 4, 5.0, "node", eulers=torch.zeros(0, 3, device=device))
    assert torch.equal(out, x0)


@pytest.mark.parametrize("mode", ["node", "edge"])
def test_gradient_matches_oracle_autograd(mode, device):
    from maloq_amd.embedding import edge_degree_embed
    lmax, N, E, C = 4, 25, 300, 16
    ei, u, eul, winv, w64 = _case(lmax, N, E, C, 9, device)
    gen = torch.Generator().manual_seed(10)
    x = torch.randn(N, (lmax + 1) ** 2, C, generator=gen)
    g = torch.randn(N if mode == "node" else E, (lmax + 1) ** 2, C, generator=gen)
    ud = u.to(device).requires_grad_()
    xd = x.to(device).requires_grad_()
    out = edge_degree_embed(xd, ud, ei.to(device), None, lmax, 5.0, mode, eulers=eul)
    out.backward(g.to(device))
    u64 = u.double().requires_grad_()
    x64 = x.double().requires_grad_()
    mapping = CoefficientMapping(lmax, 2)
    mask = CoefficientMapping(lmax, lmax).coefficient_idx(lmax, 2)
    ref = oemb.edge_degree_embedding(x64, u64, ei, w64, mapping, mask, 5.0, mode)
    ref.backward(g.double())
    scale = u64.grad.abs().max().item()
    assert (ud.grad.double().cpu() - u64.grad).abs().max().item() <= 1e-5 * scale
    if mode == "node":
        assert torch.equal(xd.grad.cpu(), g)


def test_module_forward(device):
    """EdgeDegreeEmbedding end to end: HIP RadialMLP + embedding against the
    oracle RadialMLP + oracle embedding."""
    from maloq_amd.embedding import EdgeDegreeEmbedding
    from maloq_amd.so3 import CoefficientMapping as CM
    from oracle.so2 import radial_mlp
    lmax, N, E, C = 4, 16, 200, 64   # RadialMLP output width (lmax + 1) C: a multiple of 64
    ei, _, eul, winv, w64 = _case(lmax, N, E, C, 12, device)
    torch.manual_seed(0)
    mod = EdgeDegreeEmbedding(C, lmax, 2, 90, [8, 32, 32], 5.0, 6.0, CM(lmax, 2), None).to(device)
    gen = torch.Generator().manual_seed(13)
    x_edge = torch.randn(E, 8, generator=gen)
    x = torch.zeros(N, (lmax + 1) ** 2, C)
    with torch.no_grad():
        got = mod(x.to(device), x_edge.to(device), None, ei.to(device), winv)
    lins = [m for m in mod.rad_func.net if isinstance(m, torch.nn.Linear)]
    lns = [m for m in mod.rad_func.net if isinstance(m, torch.nn.LayerNorm)]
    hidden = [(li.weight.detach().double().cpu(), li.bias.detach().double().cpu(),
               ln.weight.detach().double().cpu(), ln.bias.detach().double().cpu()) for li, ln in zip(lins[:-1], lns)]
    u = radial_mlp(x_edge.double(), hidden, lins[-1].weight.detach().double().cpu(),
                   lins[-1].bias.detach().double().cpu(), lns[0].eps)
    ref = _oracle(x, u, ei, w64, lmax, "node")
    scale = ref.abs().max().item()
    assert (got.double().cpu() - ref).abs().max().item() <= 1e-5 * scale
