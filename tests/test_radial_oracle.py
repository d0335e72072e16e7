"""CPU pin of oracle.so2.radial_mlp (the restatement of RadialMLP,
radial.py:115-142): it must equal torch's own Linear -> LayerNorm -> SiLU
stack in fp64, forward and gradients, and the build's RadialMLP module must
hold the same parameters under the same state-dict names."""
import pytest
import torch
from torch import nn

from oracle import so2 as oso2


def _reference_stack(widths, gen):
    mods = []
    for i in range(1, len(widths)):
        mods.append(nn.Linear(widths[i - 1], widths[i]))
        if i < len(widths) - 1:
            mods += [nn.LayerNorm(widths[i]), nn.SiLU()]
    net = nn.Sequential(*mods).double()
    with torch.no_grad():
        for p in net.parameters():
            p.copy_(torch.randn(p.shape, generator=gen, dtype=torch.float64) * 0.5)
    return net


def _split(net):
    lin = [m for m in net if isinstance(m, nn.Linear)]
    lns = [m for m in net if isinstance(m, nn.LayerNorm)]
    hidden = [(l.weight, l.bias, n.weight, n.bias) for l, n in zip(lin[:-1], lns)]
    return hidden, lin[-1].weight, lin[-1].bias


@pytest.mark.parametrize("widths", [(8, 64, 64, 192), (4, 32, 64), (12, 32, 64, 32, 128)])
def test_oracle_radial_matches_torch_modules(widths):
    gen = torch.Generator().manual_seed(sum(widths))
    net = _reference_stack(widths, gen)
    x = torch.randn(23, widths[0], generator=gen, dtype=torch.float64, requires_grad=True)
    ref = net(x)
    hidden, wo, bo = _split(net)
    got = oso2.radial_mlp(x, hidden, wo, bo, eps=net[1].eps)
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)
    gout = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    params = list(net.parameters())
    g_ref = torch.autograd.grad(ref, [x] + params, gout)
    g_got = torch.autograd.grad(got, [x] + params, gout)
    for a, b in zip(g_got, g_ref):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-10)


def test_oracle_radial_planted_mistake_is_caught():
    """A plausible slip (unbiased variance) changes the output measurably."""
    gen = torch.Generator().manual_seed(3)
    net = _reference_stack((8, 32, 64), gen)
    x = torch.randn(5, 8, generator=gen, dtype=torch.float64)
    hidden, wo, bo = _split(net)
    good = oso2.radial_mlp(x, hidden, wo, bo)
    w, b, g, bt = hidden[0]
    z = x @ w.T + b
    a = (z - z.mean(-1, keepdim=True)) / torch.sqrt(z.var(-1, unbiased=True, keepdim=True) + 1e-5) * g + bt
    bad = (a / (1 + torch.exp(-a))) @ wo.T + bo
    assert (good - bad).abs().max() > 1e-3
    torch.testing.assert_close(good, net(x), rtol=1e-12, atol=1e-12)


def test_module_state_dict_names_match_reference_layout():
    from maloq_amd.radial import RadialMLP
    widths = (8, 64, 64, 192)
    gen = torch.Generator().manual_seed(0)
    ref = _reference_stack(widths, gen).float()
    mod = RadialMLP(list(widths))
    assert sorted(mod.state_dict()) == sorted("net." + k for k in ref.state_dict())
    mod.net.load_state_dict(ref.state_dict())


def test_module_refuses_cpu_tensors():
    from maloq_amd.radial import RadialMLP
    mod = RadialMLP([8, 32, 64])
    with pytest.raises(ValueError, match="GPU"):
        mod(torch.zeros(3, 8))


def test_library_rejects_unsupported_widths():
    """Host-side validation (no GPU needed): widths outside the kernels' limits."""
    import ctypes
    from maloq_amd import _lib
    lib = _lib.load()
    ok = (ctypes.c_int * 4)(8, 64, 64, 1536)
    assert lib.maloq_radial_bwd_partials_floats(1, 2, ok, 1000) > 0
    for bad in [(8, 48, 64, 1536), (8, 64, 64, 1000), (6, 64, 64, 1536), (8, 256, 64, 1536), (4, 128, 64, 384)]:
        arr = (ctypes.c_int * 4)(*bad)
        assert lib.maloq_radial_bwd_partials_floats(1, 2, arr, 1000) == -1, bad
