"""The two-convolution Edgewise block (maloq_amd.edgewise, esen_block.py:37-258).

CPU: the module mirrors the reference's constructor, parameter names and
shapes, and refuses CPU tensors and a three-part message without its third part.
GPU: node and edge modes against the oracle (oracle.message, message_block
with conv2 and concat "source-target"), with the radial scales from the
oracle RadialMLP on the module's own weights, output and the gradients of x,
x_edge and every parameter (fp64 autograd through the oracle RadialMLP);
fp32 within 1e-5 of each tensor's scale."""
import pytest
import torch

from oracle import message as omsg
from oracle import rotation as orot


def _module(C=32, H=64, lmax=4, mmax=2, message_type="source-target", ecl=(8, 32, 32)):
    from maloq_amd.edgewise import Edgewise
    from maloq_amd.so3 import CoefficientMapping
    torch.manual_seed(0)
    return Edgewise(C, H, lmax, mmax, list(ecl), CoefficientMapping(lmax, mmax), None, 6.0, message_type)


def test_module_mirrors_reference_structure():
    mod = _module()
    shapes = {k: tuple(v.shape) for k, v in mod.named_parameters()}
    # conv1: input 2 C = 64, hidden 64, extra lmax H = 256 gate outputs; rad width 64 (5 + 2 * 4 + 2 * 3)
    assert shapes["so2_conv_1.fc_m0.weight"] == (5 * 64 + 4 * 64, 5 * 64)
    assert shapes["so2_conv_1.fc_m0.bias"] == (5 * 64 + 4 * 64,)
    assert shapes["so2_conv_1.so2_m_conv.0.fc.weight"] == (2 * 4 * 64, 4 * 64)
    assert shapes["so2_conv_1.so2_m_conv.1.fc.weight"] == (2 * 3 * 64, 3 * 64)
    assert shapes["so2_conv_1.rad_func.net.6.weight"] == ((5 + 4 + 3) * 64, 32)
    assert shapes["so2_conv_2.fc_m0.weight"] == (5 * 32, 5 * 64)
    assert shapes["so2_conv_2.so2_m_conv.1.fc.weight"] == (2 * 3 * 32, 3 * 64)
    assert not any(k.startswith("so2_conv_2.rad_func") for k in shapes)
    assert mod.so2_conv_1.edge_channels_list == [8, 32, 32, 12 * 64]
    assert mod.edge_channels_list == [8, 32, 32]
    assert mod.concat_size == 2 and _module(message_type="source-target-message").concat_size == 3
    with pytest.raises(ValueError):
        _module(message_type="source")


def test_module_refuses_what_is_not_built():
    from maloq_amd import _lib
    mod = _module(C=32, H=32, lmax=2)
    N, E = 4, 6
    x = torch.zeros(N, 9, 32)
    ei = torch.zeros(2, E, dtype=torch.long)
    with torch.no_grad(), pytest.raises((_lib.MaloqHipError, RuntimeError, ValueError)):   # CPU tensors
        mod(x, None, torch.zeros(E, 8), ei, None, None, "node", eulers=torch.zeros(E, 3))
    with torch.no_grad(), pytest.raises(ValueError):
        _module(C=32, H=32, lmax=2, message_type="source-target-message")(
            x, None, torch.zeros(E, 8), ei, None, None, "node", eulers=torch.zeros(E, 3))
    # shapes without kernels are refused at construction
    for kw in ({"lmax": 4, "mmax": 3}, {"lmax": 3, "mmax": 3}, {"C": 8}, {"H": 48}):
        with pytest.raises(ValueError):
            _module(**kw)
    for lmax, mmax in ((2, 2), (4, 2), (4, 4), (6, 2), (6, 6)):
        assert _module(lmax=lmax, mmax=mmax) is not None


def _oracle_conv(c):
    w0, b0, wm = c.weights()
    cpu = lambda t: t.detach().double().cpu()
    return {"w0": cpu(w0), "b0": cpu(b0), "wm": [cpu(w) for w in wm], "c_out": c.m_output_channels}


@pytest.mark.gpu
@pytest.mark.parametrize("mode,lmax,mmax,C,H,ecl,dense", [
    ("node", 2, 2, 32, 64, (8, 32, 32), False), ("edge", 2, 2, 32, 64, (8, 32, 32), False),
    ("node", 4, 2, 32, 64, (8, 32, 32), False), ("edge", 4, 2, 32, 64, (8, 32, 32), True),
    # the reference's example model shape: l_embedding_dim 128, hidden 128,
    # num_distance_basis 128, lmax = mmax = 4 (run_QM7.py:66-67,
    # training_workflow.py:508-511, esen_osh.py:189-192), its dense wigner input
    ("node", 4, 4, 128, 128, (384, 128, 128), True), ("edge", 4, 4, 128, 128, (384, 128, 128), True)])
def test_module_forward_and_gradients_match_oracle(mode, lmax, mmax, C, H, ecl, dense):
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from maloq_amd.wigner import extract_euler_angles, wigner_from_eulers
    from oracle.so2 import radial_mlp
    print(f"edgewise module case mode={mode} lmax={lmax} mmax={mmax} C={C} H={H} dense={dense}", flush=True)
    dev = torch.device("cuda:0")
    N, E = 23, 300
    mod = _module(C, H, lmax, mmax, ecl=ecl).to(dev)
    gen = torch.Generator().manual_seed(lmax)
    x = torch.randn(N, (lmax + 1) ** 2, C, generator=gen)
    src = torch.randint(0, N, (E,), generator=gen)
    dst = torch.randint(0, N - 2, (E,), generator=gen)
    ei = torch.stack([src, dst])
    x_edge = torch.randn(E, ecl[0], generator=gen)
    eul = extract_euler_angles(torch.randn(E, 3, generator=gen).to(dev), seed=5)
    xd = x.to(dev).requires_grad_()
    xe = x_edge.to(dev).requires_grad_()
    if dense:
        w = wigner_from_eulers(eul, None, lmax)
        got = mod(xd, None, xe, ei.to(dev), w, w.transpose(1, 2), mode)
    else:
        got = mod(xd, None, xe, ei.to(dev), None, None, mode, eulers=eul)
    gout = torch.randn(got.shape, generator=gen, dtype=torch.float64)
    got.backward(gout.float().to(dev))
    # oracle: the module's parameters as fp64 leaves
    params = {k: v.detach().double().cpu().requires_grad_() for k, v in mod.named_parameters()}
    rf = "so2_conv_1.rad_func.net."
    nlin = len([m for m in mod.so2_conv_1.rad_func.net if isinstance(m, torch.nn.Linear)])
    lin_idx = [i for i, m in enumerate(mod.so2_conv_1.rad_func.net) if isinstance(m, torch.nn.Linear)]
    ln_idx = [i for i, m in enumerate(mod.so2_conv_1.rad_func.net) if isinstance(m, torch.nn.LayerNorm)]
    hidden = [(params[f"{rf}{li}.weight"], params[f"{rf}{li}.bias"], params[f"{rf}{ln}.weight"],
               params[f"{rf}{ln}.bias"]) for li, ln in zip(lin_idx[:-1], ln_idx)]
    assert len(hidden) == nlin - 1
    x64, xe64 = x.double().requires_grad_(), x_edge.double().requires_grad_()
    rad = radial_mlp(xe64, hidden, params[f"{rf}{lin_idx[-1]}.weight"], params[f"{rf}{lin_idx[-1]}.bias"],
                     mod.so2_conv_1.rad_func.net[ln_idx[0]].eps)
    conv = lambda p, c: {"w0": params[f"{p}.fc_m0.weight"], "b0": params[f"{p}.fc_m0.bias"],
                         "wm": [params[f"{p}.so2_m_conv.{i}.fc.weight"] for i in range(mmax)], "c_out": c}
    e64 = eul.double().cpu()
    ref = omsg.message_block(x64, ei, (e64[:, 0], e64[:, 1], e64[:, 2]), orot.load_jd(), lmax, mmax,
                             conv("so2_conv_1", H), rad=rad, conv2=conv("so2_conv_2", C), gate=True,
                             concat="source-target", reduce=(mode == "node"))
    ref.backward(gout)
    assert got.shape == ref.shape
    pairs = [("out", got.detach(), ref.detach()), ("x", xd.grad, x64.grad), ("x_edge", xe.grad, xe64.grad)]
    pairs += [(k, v.grad, params[k].grad) for k, v in mod.named_parameters()]
    for name, a, b in pairs:
        scale = b.abs().max().item()
        assert (a.double().cpu() - b).abs().max().item() <= 1e-5 * scale, name
