"""The EXL3 directory writer (export_exl3.py; reference quantize/export_exl3.py)
on a synthetic template: byte-identical self-rebuild (--selftest-a), in-place
splicing that touches only the provided tensors' bytes, rebuilt
ARTIFACTS.sha256, key/dtype/shape checks and the reference's error cases."""
import hashlib
import json
from pathlib import Path

import pytest
import torch

import export_exl3 as ex
from exl3_template import make_template

MODULES = [(0, "self_attn.q_proj", 256, 384, 5), (0, "self_attn.k_proj", 256, 128, 7),
           (1, "mlp.down_proj", 384, 256, 4)]


@pytest.fixture()
def template(tmp_path):
    return make_template(tmp_path / "template", MODULES, seed=3)


def _fake_result(k, n, K, seed):
    g = torch.Generator().manual_seed(seed)
    return {"trellis": torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), generator=g,
                                     dtype=torch.int16),
            "suh": torch.randn(k, generator=g).half(), "svh": torch.randn(n, generator=g).half(),
            "K": K, "Wscale": 0.5}


def _blobs(d: Path):
    wm = json.loads((d / "model.safetensors.index.json").read_text())["weight_map"]
    return {k: ex.tensor_bytes(d / f, k) for k, f in wm.items()}


def _headers(d: Path):
    return {f.name: f.read_bytes()[:8 + ex.read_st_header(f)[1] - 8]
            for f in sorted(d.glob("*.safetensors"))}


def test_selftest_a_byte_identical(template, tmp_path):
    out = tmp_path / "out"
    assert ex.main(["--template", str(template), "--out", str(out), "--selftest-a",
                    "--tmpdir", str(tmp_path / "scratch")]) == 0
    for f in template.glob("*.safetensors"):
        assert (out / f.name).read_bytes() == f.read_bytes()


def test_export_splices_only_given_tensors(template, tmp_path):
    root = tmp_path / "tensors"
    res = {m: _fake_result(k, n, K, i) for i, (_, m, k, n, K) in enumerate(MODULES)}
    ex.write_quantized(root, 0, "self_attn.q_proj", res["self_attn.q_proj"])
    ex.write_quantized(root, 1, "mlp.down_proj", res["mlp.down_proj"])
    out = tmp_path / "out"
    assert ex.export(root, template, out) == 6
    before, after = _blobs(template), _blobs(out)
    assert before.keys() == after.keys()
    changed = {k for k in before if before[k] != after[k]}
    want = {f"model.language_model.layers.{lay}.{m}.{f}"
            for lay, m in ((0, "self_attn.q_proj"), (1, "mlp.down_proj"))
            for f in ("trellis", "suh", "svh")}
    assert changed == want
    for lay, m in ((0, "self_attn.q_proj"), (1, "mlp.down_proj")):
        base = f"model.language_model.layers.{lay}.{m}"
        assert after[base + ".trellis"] == res[m]["trellis"].numpy().tobytes()
        assert after[base + ".suh"] == res[m]["suh"].numpy().tobytes()
    assert _headers(out) == _headers(template)          # headers untouched
    assert ex.check_keys(template, out) == []
    # non-shard files verbatim, ARTIFACTS rebuilt over the output
    for name in ("config.json", "quantization_config.json", "tokenizer.json",
                 "model.safetensors.index.json"):
        assert (out / name).read_bytes() == (template / name).read_bytes()
    lines = (out / "ARTIFACTS.sha256").read_text().splitlines()
    files = sorted(p for p in out.iterdir() if p.is_file() and p.name != "ARTIFACTS.sha256")
    assert lines == [f"{hashlib.sha256(p.read_bytes()).hexdigest()}  {p.name}" for p in files]


def test_module_name_from_metadata(template, tmp_path):
    root = tmp_path / "tensors"
    p = ex.write_quantized(root, 0, "kproj_file", _fake_result(256, 128, 7, 9),
                           extra_meta={"module": "self_attn.k_proj"})
    assert p.name == "kproj_file.safetensors"
    got = ex.collect_inputs(root)
    assert sorted(got) == [f"model.language_model.layers.0.self_attn.k_proj.{f}"
                           for f in ("suh", "svh", "trellis")]
    assert got["model.language_model.layers.0.self_attn.k_proj.trellis"][:2] == \
        ("I16", [16, 8, 112])


def test_export_errors(template, tmp_path):
    from safetensors.torch import save_file
    # shape mismatch (K=4 trellis into a K=5 slot)
    root = tmp_path / "bad_shape"
    ex.write_quantized(root, 0, "self_attn.q_proj", _fake_result(256, 384, 4, 1))
    with pytest.raises(ValueError, match="shape"):
        ex.export(root, template, tmp_path / "o1")
    # dtype mismatch (fp32 suh)
    root = tmp_path / "bad_dtype"
    r = _fake_result(256, 384, 5, 1)
    (root / "L00").mkdir(parents=True)
    save_file({"trellis": r["trellis"], "suh": r["suh"].float(), "svh": r["svh"]},
              str(root / "L00" / "self_attn.q_proj.safetensors"))
    with pytest.raises(ValueError, match="dtype"):
        ex.export(root, template, tmp_path / "o2")
    # key not in the template
    root = tmp_path / "unknown"
    ex.write_quantized(root, 7, "self_attn.q_proj", _fake_result(256, 384, 5, 1))
    with pytest.raises(KeyError, match="not in the template"):
        ex.export(root, template, tmp_path / "o3")
    # missing field
    root = tmp_path / "missing"
    (root / "L00").mkdir(parents=True)
    save_file({"trellis": r["trellis"], "suh": r["suh"]},
              str(root / "L00" / "self_attn.q_proj.safetensors"))
    with pytest.raises(KeyError, match="svh"):
        ex.collect_inputs(root)


def test_check_keys_reports_problems(template, tmp_path):
    out = tmp_path / "out"
    ex.main(["--template", str(template), "--out", str(out), "--selftest-a"])
    idx = json.loads((out / "model.safetensors.index.json").read_text())
    gone = "model.language_model.layers.1.mlp.down_proj.svh"
    del idx["weight_map"][gone]
    (out / "model.safetensors.index.json").write_text(json.dumps(idx))
    assert ex.check_keys(template, out) == [(gone, "missing-from-index")]


@pytest.mark.parametrize("K", (2, 5, 7))
def test_independent_decoder_vs_oracle(oracle_mod, K):
    """The --selftest-b decoder (torch integer ops, no GPU kernel) unpacks
    and decodes random trellis streams exactly as the oracle does
    (quantize.py:381-415), and its weight is from_inner of that decode."""
    import quantize as xq
    g = torch.Generator().manual_seed(K)
    tr = torch.randint(-32768, 32768, (8, 8, 16 * K), generator=g, dtype=torch.int16)
    st = ex._states_from_stream(tr.view(-1, 16 * K), K)
    assert torch.equal(st, torch.from_numpy(oracle_mod.unpack(tr.view(-1, 16 * K).numpy(), K))
                       .long())
    suh, svh = torch.randn(128, generator=g).half(), torch.randn(128, generator=g).half()
    w = ex.weight_orig_torch(tr, suh, svh, K, device="cpu")
    lut = oracle_mod.code_lut("exl3_mul1")
    inner = torch.from_numpy(oracle_mod.decode(tr.numpy(), lut, K))
    h = xq.hadamard128("cpu", torch.float32)
    assert torch.equal(w, xq.from_inner(inner, suh, svh, h))
