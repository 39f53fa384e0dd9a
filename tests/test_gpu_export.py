"""C4 mixed-K fused qkv on the GPU: quantize q (K=5), k and v (K=7) with
channel scales, write them as EXL3 tensors, splice them into a template,
reconstruct each written tensor (HIP decode + inverse incoherence) and check
it against the quantizer's W_hat bit for bit (export_exl3.py --selftest-b),
then run the fused M=1 GEMV y = x [Wq; Wk; Wv]^T in fp16 against fp32
(relative error < 0.02, the tolerance of serve/tests/check_mixedk.py:119-126).
Sizes are the C4 recipe shrunk 8x (d = 640)."""
import json

import pytest
import torch

import export_exl3 as ex
import quantize as xq
import workloads as wl
from exl3_template import make_template

pytestmark = pytest.mark.gpu


def test_c4_qkv_write_reconstruct_gemv(tmp_path):
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    w = wl.c4(scale=8, device="cuda")
    H = w["H"].cuda()
    root, specs, members = tmp_path / "tensors", [], []
    for m in w["members"]:
        print(f"case c4/8 {m['module']} K={m['K']} {tuple(m['W'].shape)}", flush=True)
        r = xq.quantize_linear(m["W"].float().cuda(), H, K=m["K"], device="cuda",
                               channel_scales=True)
        ex.write_quantized(root, 0, m["module"], r)
        torch.save(r["W_hat"], tmp_path / f"{m['module']}.pt")
        specs.append(f"L00/{m['module']}|{tmp_path / (m['module'] + '.pt')}")
        members.append((m, r))
    tpl = make_template(tmp_path / "tpl", [(0, m["module"], m["W"].shape[1], m["W"].shape[0],
                                            m["K"]) for m in w["members"]])
    out = tmp_path / "out"
    assert ex.export(root, tpl, out) == 9
    assert ex.check_keys(tpl, out) == []
    res = ex.selftest_b(tpl, out, specs, device="cuda")
    assert all(eq for _, eq, _ in res), res

    # fused GEMV over the reconstructed members, fp16 on the GPU vs fp32 on the CPU
    wm = json.loads((out / "model.safetensors.index.json").read_text())["weight_map"]
    from safetensors import safe_open
    Ws = []
    for m, r in members:
        base = f"model.language_model.layers.0.{m['module']}"
        got = {}
        for fld in ("trellis", "suh", "svh"):
            with safe_open(str(out / wm[f"{base}.{fld}"]), framework="pt") as f:
                got[fld] = f.get_tensor(f"{base}.{fld}")
        tr, suh, svh = got["trellis"], got["suh"], got["svh"]
        assert tr.shape[-1] == 16 * m["K"]
        Ws.append(ex.weight_orig(tr, suh, svh, m["K"], device="cuda").t())   # [out, in]
    W_cat = torch.cat(Ws, 0)
    x = w["x"].cuda()
    y16 = (x @ W_cat.half().t()).float().cpu()
    y32 = x.float().cpu() @ W_cat.cpu().t()
    rel = float((y16.double() - y32.double()).norm() / y32.double().norm())
    assert rel < 0.02, rel
    # and the quantized layer tracks the original one
    W_orig = torch.cat([m["W"].float() for m in w["members"]], 0)
    rel_q = float((y32 - x.float().cpu() @ W_orig.t()).norm() / (x.float().cpu() @ W_orig.t()).norm())
    assert rel_q < 0.2, rel_q
