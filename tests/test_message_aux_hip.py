"""Weight packing (maloq_message_pack) and the fc_m0 bias-gradient column sums
(maloq_message_colsum) on the GPU, against host restatements: the packing is a
gather + round-to-nearest-even conversion (bit-exact against torch's CPU
gather and cast), the column sums a plain sum (fp64 reference, fp32 bar 1e-5
relative; bit-identical across repeated calls)."""
import numpy as np
import pytest
import torch

from maloq_amd import _lib
from maloq_amd import message as M

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def device():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("lmax,mmax,gate,mode", [(2, 2, False, 0), (4, 2, True, 0), (4, 2, True, 1),
                                                 (6, 2, False, 1)])
def test_pack_matches_host_gather(lmax, mmax, gate, mode, dtype, device):
    print(f"pack case lmax={lmax} gate={gate} mode={mode} dtype={dtype}", flush=True)
    c_in, c_out = 32, 64
    gen = torch.Generator().manual_seed(lmax + 10 * mode)
    extra = lmax * c_out if gate else 0
    w0 = torch.randn(extra + (lmax + 1) * c_out, (lmax + 1) * c_in, generator=gen)
    wm = [torch.randn(2 * (lmax - m + 1) * c_out, (lmax - m + 1) * c_in, generator=gen)
          for m in range(1, mmax + 1)]
    code = M.DTYPE_CODE[dtype]
    idx, total = M._pack_index(code, lmax, mmax, gate, c_in, c_out, mode)
    flat = torch.cat([w0.reshape(-1)] + [w.reshape(-1) for w in wm])
    assert flat.numel() == total
    want = flat[torch.from_numpy(idx)].to(dtype)
    got = M.pack_weights(w0.to(device), [w.to(device) for w in wm], lmax, mmax, gate, c_in, c_out, dtype,
                         mode).cpu()
    assert got.dtype == dtype and got.shape == want.shape
    assert torch.equal(got.view(torch.uint8 if dtype == torch.float32 else torch.int16).flatten(),
                       want.view(torch.uint8 if dtype == torch.float32 else torch.int16).flatten())


def _colsum(rows, row0, nrows, E):
    lib = _lib.load()
    c = rows.shape[2]
    parts = torch.empty(max(1, lib.maloq_message_colsum_partials_floats(nrows, c, E)), device=rows.device)
    out = torch.full((nrows * c,), float("nan"), device=rows.device)
    _lib.call("maloq_message_colsum", M.DTYPE_CODE[rows.dtype], _lib.ptr(rows), rows.shape[1], row0, nrows, c, E,
              _lib.ptr(parts), _lib.ptr(out), _lib.stream_of(rows.device))
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("gate", [False, True])
def test_pack_both_equals_the_two_packings(gate, dtype, device):
    """mode "both" (one launch) gives bit-for-bit the forward and transposed
    packings of two separate launches, each slice 16-byte aligned."""
    lmax, mmax, c_in, c_out = 4, 2, 64, 32
    gen = torch.Generator().manual_seed(5 + int(gate))
    extra = lmax * c_out if gate else 0
    w0 = torch.randn((lmax + 1) * c_out + extra, (lmax + 1) * c_in, generator=gen).to(device)
    wm = [torch.randn(2 * (lmax - m + 1) * c_out, (lmax - m + 1) * c_in, generator=gen).to(device)
          for m in range(1, mmax + 1)]
    a, b = M.pack_weights(w0, wm, lmax, mmax, gate, c_in, c_out, dtype, "both")
    assert torch.equal(a, M.pack_weights(w0, wm, lmax, mmax, gate, c_in, c_out, dtype, 0))
    assert torch.equal(b, M.pack_weights(w0, wm, lmax, mmax, gate, c_in, c_out, dtype, 1))
    assert a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("E", [0, 1, 63, 64, 65, 1000, 4097, 300001])
def test_colsum_matches_fp64(E, dtype, device):
    print(f"colsum case E={E} dtype={dtype}", flush=True)
    rpe, c, row0, nrows = (11, 64, 3, 5) if E < 10000 else (6, 16, 1, 4)
    gen = torch.Generator().manual_seed(E)
    rows = torch.randn(E + 7, rpe, c, generator=gen).to(dtype)  # rows past E must be ignored
    rows[E:] = 1e30
    d = rows.to(device)
    got = _colsum(d, row0, nrows, E).cpu().double()
    ref = rows[:E, row0: row0 + nrows].double().sum(0).reshape(-1)
    scale = rows[:E, row0: row0 + nrows].double().abs().sum(0).reshape(-1).clamp_min(1.0)
    assert torch.all((got - ref).abs() <= 1e-5 * scale), float(((got - ref).abs() / scale).max())
    again = _colsum(d, row0, nrows, E).cpu().double()
    assert torch.equal(got, again)


def test_colsum_rejects_bad_rows(device):
    rows = torch.zeros(4, 3, 12, device=device)
    with pytest.raises(_lib.MaloqHipError, match="row range"):
        _colsum(rows, 2, 2, 4)
    rows = torch.zeros(4, 3, 12, device=device, dtype=torch.bfloat16)
    with pytest.raises(_lib.MaloqHipError, match="multiple of 8"):
        _colsum(rows, 0, 2, 4)


def test_bias_grad_is_column_sum_of_saved_rows(device):
    """message_weight_grad's db0: gate rows first, then the m = 0 rows."""
    lmax, mmax, c_in, c_out, E = 4, 2, 32, 64, 777
    kept = M.kept_rows(lmax, mmax)
    n = int(_lib.load().maloq_message_edge_rows(E))
    gen = torch.Generator().manual_seed(5)
    dz = torch.zeros(n, kept + lmax, c_out)
    dz[:E] = torch.randn(E, kept + lmax, c_out, generator=gen)
    y = torch.zeros(n, kept, c_in)
    y[:E] = torch.randn(E, kept, c_in, generator=gen)
    dzb, yb = dz.to(torch.bfloat16), y.to(torch.bfloat16)
    _, _, db0 = M.message_weight_grad(dzb.to(device), yb.to(device), lmax, mmax, c_out, c_in, num_edges=E,
                                      gate=True)
    ref = torch.cat([dzb[:E, kept:].double().sum(0).reshape(-1), dzb[:E, : lmax + 1].double().sum(0).reshape(-1)])
    np.testing.assert_allclose(db0.cpu().double().numpy(), ref.numpy(), rtol=1e-5, atol=1e-4)
