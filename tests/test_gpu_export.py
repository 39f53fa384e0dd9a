"""C4 mixed-K fused qkv at full size on the GPU: q 6144x5120 (K=5), k and v
1024x5120 (K=7), one shared Hessian, channel scales, quantized in one
quantize_linear_group sweep, written as EXL3 tensors and spliced into a
template; then, from the written files alone:

  * --selftest-b: the writer's decoder that is independent of the GPU kernels
    (torch integer ops on the bit stream) reproduces each saved W_hat bit for
    bit (export_exl3.py:195-222 of the reference);
  * an independent reconstruction for the check: the C oracle's decode and
    the inverse incoherence transform in fp64 on the CPU.  The GPU weight
    (HIP decode, fp32 transform: weight_orig) agrees with it within the fp32
    rounding bound of the two 128-long Hadamard products;
  * the fused M=1 GEMV y = x [Wq; Wk; Wv]^T with an fp16 activation: fp16
    weights on the GPU against the fp64 weight, relative error < 0.02
    (serve/tests/check_mixedk.py:94-126).
"""
import json

import numpy as np
import pytest
import torch

import export_exl3 as ex
import quantize as xq
import workloads as wl
from exl3_template import make_template

pytestmark = pytest.mark.gpu


def _from_inner_fp64(inner: np.ndarray, suh: np.ndarray, svh: np.ndarray) -> np.ndarray:
    """diag(suh) B_k W_inner B_n diag(svh) in fp64 (B: block-128 Sylvester
    Hadamard / sqrt(128)), [k, n]."""
    h = np.ones((1, 1))
    while h.shape[0] < 128:
        h = np.block([[h, h], [h, -h]])
    h = h / np.sqrt(128.0)
    k, n = inner.shape
    w = np.matmul(h, inner.reshape(k // 128, 128, n)).reshape(k, n) * suh[:, None]
    return np.matmul(w.reshape(k, n // 128, 128), h).reshape(k, n) * svh[None, :]


def _fp32_bound(inner: np.ndarray, suh: np.ndarray, svh: np.ndarray) -> np.ndarray:
    """Worst-case fp32 error of the transform: two 128-term dot products and
    two scalings, (2*128 + 4) u |suh| (|B| |W_inner| |B|) |svh| with
    |B| = 1/sqrt(128) everywhere, i.e. the block's sum of |W_inner| / 128."""
    k, n = inner.shape
    blk = np.abs(inner).reshape(k // 128, 128, n // 128, 128).sum(axis=(1, 3)) / 128.0
    mag = np.repeat(np.repeat(blk, 128, axis=0), 128, axis=1)
    return (2 * 128 + 4) * 2.0 ** -24 * np.abs(suh)[:, None] * mag * np.abs(svh)[None, :]


def test_c4_full_size_write_reconstruct_gemv(tmp_path, oracle_mod):
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    w = wl.c4(device="cuda")
    H = w["H"].cuda()
    Ks = [m["K"] for m in w["members"]]
    print(f"case c4 full size K={Ks}", flush=True)
    rs = xq.quantize_linear_group([m["W"].float().cuda() for m in w["members"]], H, K=Ks,
                                  device="cuda", channel_scales=True)
    root, specs = tmp_path / "tensors", []
    for m, r in zip(w["members"], rs):
        ex.write_quantized(root, 0, m["module"], r)
        torch.save(r["W_hat"], tmp_path / f"{m['module']}.pt")
        specs.append(f"L00/{m['module']}|{tmp_path / (m['module'] + '.pt')}")
    tpl = make_template(tmp_path / "tpl", [(0, m["module"], m["W"].shape[1], m["W"].shape[0],
                                            m["K"]) for m in w["members"]])
    out = tmp_path / "out"
    assert ex.export(root, tpl, out) == 9
    assert ex.check_keys(tpl, out) == []
    res = ex.selftest_b(tpl, out, specs, device="cuda")
    print(f"selftest-b {res}", flush=True)
    assert all(eq for _, eq, _ in res), res

    lut = oracle_mod.code_lut("exl3_mul1")
    wm = json.loads((out / "model.safetensors.index.json").read_text())["weight_map"]
    W64, W32 = [], []
    for m in w["members"]:
        base = f"model.language_model.layers.0.{m['module']}"
        f = {fld: ex._StFile(out / wm[f"{base}.{fld}"]).tensor(f"{base}.{fld}")
             for fld in ("trellis", "suh", "svh")}
        inner = oracle_mod.decode(f["trellis"].numpy(), lut, m["K"]).astype(np.float64)
        suh = f["suh"].float().numpy().astype(np.float64)
        svh = f["svh"].float().numpy().astype(np.float64)
        w64 = _from_inner_fp64(inner, suh, svh)                          # [in, out]
        w32 = ex.weight_orig(f["trellis"], f["suh"], f["svh"], m["K"], device="cuda")
        err = np.abs(w32.cpu().numpy().astype(np.float64) - w64)
        bound = _fp32_bound(inner, suh, svh)
        print(f"{m['module']}: max |w32 - w64| {err.max():.3e}, worst err/bound "
              f"{(err / np.maximum(bound, 1e-300)).max():.3e}", flush=True)
        assert (err <= bound).all()
        W64.append(w64.T)
        W32.append(w32.t())
    x = w["x"].cuda()                                                    # fp16 [1, in]
    W64c = np.concatenate(W64, 0)                                        # [out, in]
    y64 = x.double().cpu().numpy() @ W64c.T
    y16 = (x @ torch.cat(W32, 0).half().t()).double().cpu().numpy()
    rel = float(np.linalg.norm(y16 - y64) / np.linalg.norm(y64))
    print(f"GEMV fp16 vs fp64 weight: rel {rel:.3e}", flush=True)
    assert rel < 0.02
    # the quantized layer tracks the original one
    W_orig = torch.cat([m["W"].double() for m in w["members"]], 0).numpy()
    y_o = x.double().cpu().numpy() @ W_orig.T
    rel_q = float(np.linalg.norm(y64 - y_o) / np.linalg.norm(y_o))
    print(f"GEMV quantized vs original: rel {rel_q:.3e}", flush=True)
    assert rel_q < 0.2
