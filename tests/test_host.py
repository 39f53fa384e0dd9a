"""Host-side logic of the quantize.py mirror, checked on CPU (no GPU needed).

The incoherence transform, codebook tables, sign vectors, block-LDL and the
error behaviour of the public API are compared with the reference's golden
vectors and with closed forms (quantize.py:52-437, 969-1058).
"""
import numpy as np
import pytest
import torch

from conftest import load_golden


@pytest.fixture(scope="module")
def xq():
    import quantize
    return quantize


def test_get_lut_golden(xq, oracle_mod):
    g = load_golden("lut_mul1.npz")
    np.testing.assert_array_equal(xq.get_lut("exl3_mul1").numpy(), g["lut"])
    for name in ("exl3_3inst", "exl3_mcg", "qtip_1mad"):
        np.testing.assert_array_equal(xq.get_lut(name).numpy(), oracle_mod.code_lut(name))
    with pytest.raises(KeyError):
        xq.get_lut("xe_ih2x2")


def test_get_lut_small_L(xq, oracle_mod):
    np.testing.assert_array_equal(xq.get_lut("exl3_mul1", 8).numpy(),
                                  oracle_mod.code_lut("exl3_mul1", 8))


def test_host_buffers(xq):
    """The background-allocated result buffers have the requested shapes
    and dtypes, are contiguous host tensors, and are handed out once."""
    specs = [((40, 1024), torch.float32), ((3, 2, 48), torch.int16), ((0,), torch.float32)]
    bufs = xq._HostBuffers(specs)
    for i, (shape, dt) in enumerate(specs):
        t = bufs.take(i)
        assert t.shape == shape and t.dtype == dt and t.is_contiguous()
        assert t.device.type == "cpu"
        assert bufs.take(i) is None


def test_perm_golden(xq):
    np.testing.assert_array_equal(xq.tensor_core_perm().numpy(),
                                  load_golden("lut_mul1.npz")["perm"])


def test_sign_vec_golden(xq):
    g = load_golden("sign_vec.npz")
    for n in (128, 256):
        for s in (20261011, 20261012, 7):
            np.testing.assert_array_equal(xq.sign_vec(n, s).numpy(), g[f"sign_{n}_{s}"])


def test_cached_tables_hand_out_own_tensors(xq):
    """get_lut and sign_vec compute their values once per key: writing into
    a returned tensor must not change what later calls return."""
    g = load_golden("sign_vec.npz")
    v = xq.sign_vec(256, 7)
    v.fill_(3.0)
    np.testing.assert_array_equal(xq.sign_vec(256, 7).numpy(), g["sign_256_7"])
    lut = xq.get_lut("exl3_mul1", 16)
    want = lut.clone()
    lut.zero_()
    assert torch.equal(xq.get_lut("exl3_mul1", 16), want)
    assert not xq._code_table("exl3_mul1", 16).flags.writeable


def test_hadamard_closed_form(xq):
    h = xq.hadamard128(None, torch.float64)
    assert torch.allclose(h @ h, torch.eye(128, dtype=torch.float64), atol=1e-14)
    assert torch.equal(h, h.t())
    assert torch.all(h.abs() == 1 / np.sqrt(128))


def test_incoherence_roundtrip(xq):
    g = torch.Generator().manual_seed(1)
    W = torch.randn(256, 384, generator=g)
    su = xq.sign_vec(256, 1).half()
    sv = xq.sign_vec(384, 2).half()
    h = xq.hadamard128(None, torch.float32)
    Wi = xq.to_inner(W, su, sv, h)
    assert torch.allclose(xq.from_inner(Wi, su, sv, h), W, atol=1e-5)
    # the rotated Gram of x equals the Gram of the rotated inputs
    X = torch.randn(64, 256, generator=g, dtype=torch.float64)
    H = (X.t() @ X).float()
    G = xq.rotate_hessian(H, su, h)
    Xr = xq.had_right(X.float() * su.float(), h)
    assert torch.allclose(G, Xr.t() @ Xr, rtol=1e-4, atol=1e-3)


def test_block_ldl_properties(xq):
    g = torch.Generator().manual_seed(3)
    A = torch.randn(96, 96, generator=g, dtype=torch.float64)
    G = A @ A.t() / 96 + 0.1 * torch.eye(96, dtype=torch.float64)
    L, D = xq.block_LDL(G.clone(), 16)
    m = 6
    Dfull = torch.block_diag(*D)
    assert torch.allclose(L @ Dfull @ L.t(), G, atol=1e-10)
    Lb = L.view(m, 16, m, 16)
    for i in range(m):
        assert torch.equal(Lb[i, :, i, :], torch.eye(16, dtype=L.dtype))
        for j in range(i + 1, m):
            assert not Lb[i, :, j, :].any()
    with pytest.raises(RuntimeError):
        xq.block_LDL(-torch.eye(32, dtype=torch.float64), 16)


def test_factor_fallback_damping(xq):
    """A Gram that is not SPD in fp32 is retried in fp64 with extra damping
    (quantize.py:815-835); a non-finite Gram raises."""
    G = torch.eye(32)
    G[0, 0] = -1e-3
    L = xq._factor_hessian(G.clone())
    assert torch.isfinite(L).all()
    bad = torch.eye(32)
    bad[1, 1] = float("nan")
    with pytest.raises(RuntimeError):
        xq._factor_hessian(bad)


def test_prepare_incoherence_golden(xq):
    e = load_golden("e2e_128.npz")
    prep = xq.prepare_incoherence(torch.from_numpy(e["W"]), torch.from_numpy(e["H_ar"]),
                                  channel_scales=True)
    np.testing.assert_array_equal(prep["Wt"].numpy(), e["prep_Wt"])
    np.testing.assert_array_equal(prep["G"].numpy(), e["prep_G"])
    np.testing.assert_array_equal(prep["suh"].numpy(), e["prep_suh"])
    np.testing.assert_array_equal(prep["svh"].numpy(), e["prep_svh"])


def test_metrics(xq):
    W = torch.randn(8, 16)
    assert xq.rel_mse(W, W) == 0.0
    assert abs(xq.rel_mse(W, 2 * W) - 1.0) < 1e-6
    H = torch.eye(16)
    assert abs(xq.hessian_weighted_err(W, 0 * W, H) - 1.0) < 1e-6


def test_unsupported_variants_raise(xq):
    lut = xq.get_lut("exl3_mul1")
    X = torch.zeros(256, 2)
    with pytest.raises(NotImplementedError):
        xq.viterbi(X, lut, 4, 16, emit_mode="addmm")
    with pytest.raises(NotImplementedError):
        xq.viterbi(X, lut, 4, 16, V=2)
    with pytest.raises(NotImplementedError):
        xq.quantize_seq_tailbite(X, xq.get_lut("exl3_mul1", 12), 4, 12)
    with pytest.raises(NotImplementedError):        # a table of no supported code
        xq.quantize_seq_tailbite(X, xq.get_lut("qtip_1mad") * 2, 4, 16)
    with pytest.raises(NotImplementedError):
        xq.quantize_seq_tailbite(torch.zeros(128, 2), lut, 4, 16)
    with pytest.raises(ValueError):
        xq.ldlq_viterbi(torch.zeros(16, 16), None, lut, 4, 16, backend="dual")
    with pytest.raises(ValueError):
        xq.ldlq_viterbi(torch.zeros(16, 16), None, lut, 4, 16, schedule="rows")
    # group members must share the input dimension (one Hessian)
    with pytest.raises(ValueError):
        xq.quantize_linear_group([torch.zeros(128, 256), torch.zeros(128, 128)], None)
    with pytest.raises(ValueError):
        xq.quantize_linear_group([], None)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_no_cpu_fallback(xq):
    """Without a HIP device the trellis path raises instead of falling back."""
    lut = xq.get_lut("exl3_mul1")
    with pytest.raises(RuntimeError):
        xq.quantize_seq_tailbite(torch.zeros(256, 2), lut, 4, 16)
    with pytest.raises(RuntimeError):
        xq.quantize_linear(torch.randn(128, 128), None, K=4)
    with pytest.raises(RuntimeError):
        xq.ldlq_viterbi(torch.randn(32, 32), None, lut, 4, 16, schedule="chain")
