#!/usr/bin/env python3
"""export_exl3.py -- write trellis-quantized tensors into an EXL3 model
directory (the writer of the reference, quantize/export_exl3.py).

Inputs (--tensors ROOT) follow the reference's per-tensor layout
(export_exl3.py:3-8):

    ROOT/L{nn}/{module}.safetensors   trellis int16 [k/16, n/16, 16K],
                                      suh fp16 [k], svh fp16 [n]
    ROOT/L{nn}/{module}.json          optional metadata; "module" overrides
                                      the file stem, other fields ("K",
                                      "Wscale", ...) are informational

and map to the template keys model.language_model.layers.{nn}.{module}.{field}.
The template (--template) is an EXL3 model directory (index + shards).  The
output (--out) is the template with every provided tensor's bytes replaced in
place inside its shard -- headers untouched, so writing the template's own
tensors back gives byte-identical shards -- all other files copied verbatim
and ARTIFACTS.sha256 rebuilt over the output files.

Checks (export_exl3.py:150-245): --selftest-a rebuilds the template from its
own tensors and compares the shard bytes; --selftest-b decodes written
tensors (HIP decode, then the inverse incoherence transform) and compares
them with a saved W_hat; --check-keys verifies that every template key is in
the output with its dtype and shape.

write_quantized() is the harness side: it stores one quantize_linear result
in the input layout.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import shutil
import struct
import sys
import tempfile
from pathlib import Path

# bytes per element of the safetensors dtypes
ST_DTYPES = {"F64": 8, "F32": 4, "F16": 2, "BF16": 2, "I64": 8, "I32": 4,
             "I16": 2, "I8": 1, "U8": 1, "BOOL": 1}
QUANT_FIELDS = ("trellis", "suh", "svh")
LAYER_PREFIX = "model.language_model.layers."

_NUMPY_TO_ST = {"int16": "I16", "float16": "F16", "float32": "F32", "int32": "I32",
                "int64": "I64", "uint8": "U8", "bool": "BOOL"}
_ST_TO_TORCH = {"F16": "float16", "I16": "int16", "F32": "float32", "I32": "int32",
                "BF16": "bfloat16", "I64": "int64", "U8": "uint8", "BOOL": "bool"}


# ------------------------------------------------------------ safetensors
def read_st_header(path):
    """(header dict, byte offset of the data section) of a safetensors file:
    an 8-byte little-endian header length, the JSON header, then the data."""
    with open(path, "rb") as f:
        (hlen,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(hlen))
    return header, 8 + hlen


def tensor_bytes(path, key):
    """Raw bytes of tensor `key` inside safetensors file `path`."""
    header, base = read_st_header(path)
    lo, hi = header[key]["data_offsets"]
    with open(path, "rb") as f:
        f.seek(base + lo)
        return f.read(hi - lo)


def _layer_key(nn, module, field):
    return f"{LAYER_PREFIX}{int(nn)}.{module}.{field}"


# ------------------------------------------------------------------ inputs
def collect_inputs(tensors_root):
    """Every quantized tensor under ROOT/L*/ -> {template key: (st dtype,
    shape, raw bytes)}.  A file missing one of trellis/suh/svh raises
    KeyError; an unsupported dtype raises ValueError."""
    from safetensors import safe_open
    found = {}
    for st_path in sorted(Path(tensors_root).glob("L*/*.safetensors")):
        nn = int(st_path.parent.name[1:])
        module = st_path.stem
        meta_path = st_path.with_suffix(".json")
        if meta_path.exists():
            module = json.loads(meta_path.read_text()).get("module", module)
        with safe_open(str(st_path), framework="np") as f:
            keys = set(f.keys())
            missing = [fld for fld in QUANT_FIELDS if fld not in keys]
            if missing:
                raise KeyError(f"{st_path}: missing key {missing[0]!r} (has {sorted(keys)})")
            for fld in QUANT_FIELDS:
                arr = f.get_tensor(fld)
                st_dtype = _NUMPY_TO_ST.get(str(arr.dtype))
                if st_dtype is None:
                    raise ValueError(f"{st_path}:{fld} dtype {arr.dtype}")
                found[_layer_key(nn, module, fld)] = (st_dtype, list(arr.shape),
                                                      arr.tobytes(order="C"))
    return found


def write_quantized(root, layer: int, module: str, result: dict, extra_meta=None) -> Path:
    """Store one quantize_linear result (trellis, suh, svh) as
    ROOT/L{layer:02d}/{module}.safetensors plus its .json metadata."""
    import torch
    from safetensors.torch import save_file
    ldir = Path(root) / f"L{int(layer):02d}"
    ldir.mkdir(parents=True, exist_ok=True)
    path = ldir / f"{module}.safetensors"
    tensors = {"trellis": result["trellis"].to("cpu", torch.int16).contiguous(),
               "suh": result["suh"].to("cpu", torch.float16).contiguous(),
               "svh": result["svh"].to("cpu", torch.float16).contiguous()}
    save_file(tensors, str(path))
    meta = {"module": module, "K": int(result.get("K", tensors["trellis"].shape[-1] // 16))}
    for k in ("Wscale", "code", "channel_scales", "use_ldlq"):
        if k in result:
            meta[k] = result[k]
    meta.update(extra_meta or {})
    path.with_suffix(".json").write_text(json.dumps(meta))
    return path


# ------------------------------------------------------------------ export
def _sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            chunk = f.read(1 << 24)
            if not chunk:
                break
            h.update(chunk)
    return h.hexdigest()


def export(tensors_root, template, outdir):
    """Splice the quantized tensors under tensors_root into a copy of the
    template directory; returns the number of tensors replaced."""
    template, outdir = Path(template), Path(outdir)
    weight_map = json.loads((template / "model.safetensors.index.json").read_text())["weight_map"]
    inputs = collect_inputs(tensors_root)
    unknown = [k for k in inputs if k not in weight_map]
    if unknown:
        raise KeyError(f"input key {unknown[0]} not in template index")

    by_shard: dict = {}
    for key, blob in inputs.items():
        by_shard.setdefault(weight_map[key], {})[key] = blob

    outdir.mkdir(parents=True, exist_ok=True)
    shards = sorted(set(weight_map.values()))
    written = set()
    for shard in shards:
        header, base = read_st_header(template / shard)
        repl = by_shard.get(shard, {})
        # validate everything for this shard before writing any byte of it
        for key, (dt, shape, raw) in repl.items():
            ent = header[key]
            if ent["dtype"] != dt:
                raise ValueError(f"{key}: dtype {dt} != template {ent['dtype']}")
            if ent["shape"] != shape:
                raise ValueError(f"{key}: shape {shape} != template {ent['shape']}")
            lo, hi = ent["data_offsets"]
            if hi - lo != len(raw):
                raise ValueError(f"{key}: nbytes mismatch")
        shutil.copyfile(template / shard, outdir / shard)
        if repl:
            with open(outdir / shard, "r+b") as f:
                for key, (_, _, raw) in repl.items():
                    f.seek(base + header[key]["data_offsets"][0])
                    f.write(raw)
                    written.add(key)
    if written != set(inputs):
        raise RuntimeError(f"keys not written: {sorted(set(inputs) - written)}")

    # configs, tokenizer, index, licence ...: verbatim
    shard_set = set(shards)
    for item in template.iterdir():
        if item.is_file() and item.name not in shard_set and item.name != "ARTIFACTS.sha256":
            shutil.copyfile(item, outdir / item.name)

    lines = [f"{_sha256(item)}  {item.name}" for item in sorted(outdir.iterdir())
             if item.is_file() and item.name != "ARTIFACTS.sha256"]
    (outdir / "ARTIFACTS.sha256").write_text("\n".join(lines) + "\n")
    return len(written)


# ------------------------------------------------------------------ checks
def selftest_a(template, workdir, only_keys=None):
    """Extract the template's own decoder-layer quantized tensors into the
    input layout under workdir/tensors; returns (root, files written).
    Keys outside model.language_model.layers.* (lm_head, mtp.*) have no input
    layout and keep the template bytes."""
    import torch
    from safetensors.torch import save_file
    template = Path(template)
    weight_map = json.loads((template / "model.safetensors.index.json").read_text())["weight_map"]
    root = Path(workdir) / "tensors"
    files: dict = {}
    for key, shard in weight_map.items():
        if not key.endswith(QUANT_FIELDS) or not key.startswith(LAYER_PREFIX):
            continue
        if only_keys is not None and key not in only_keys:
            continue
        parts = key[len(LAYER_PREFIX):].split(".")
        nn, module, field = parts[0], ".".join(parts[1:-1]), parts[-1]
        header, _ = read_st_header(template / shard)
        ent = header[key]
        dtype = getattr(torch, _ST_TO_TORCH[ent["dtype"]])
        raw = bytearray(tensor_bytes(template / shard, key))
        t = torch.frombuffer(raw, dtype=dtype).reshape(ent["shape"]).clone()
        path = root / f"L{nn}" / f"{module}.safetensors"
        files.setdefault(path, {})[field] = t
    for path, tensors in files.items():
        path.parent.mkdir(parents=True, exist_ok=True)
        save_file(tensors, str(path))
        K = int(tensors["trellis"].shape[-1]) // 16 if "trellis" in tensors else 4
        path.with_suffix(".json").write_text(json.dumps({"module": path.stem, "K": K}))
    return root, len(files)


def weight_orig(trellis, suh, svh, K: int, code: str = "exl3_mul1", device=None):
    """Original-basis weight [k, n] fp32 of one EXL3 tensor: the HIP trellis
    decode followed by diag(suh) B W_inner B diag(svh) (the inverse
    incoherence transform, quantize.py:158-164).  quantize_linear builds its
    W_hat with the same operations, so W_hat == weight_orig(...).t() when
    both run on the same device."""
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import hip_backend as hb
    import quantize as xq
    dev = torch.device(device) if device is not None else torch.device("cuda")
    tr = trellis.to("cuda", torch.int16).contiguous()
    w_inner = hb.decode(tr, int(K), code=hb.code_name(code)).to(dev)
    h = xq.hadamard128(dev, torch.float32)
    return xq.from_inner(w_inner, suh.to(dev), svh.to(dev), h)


def selftest_b(template, outdir, what_if, device=None):
    """For each "L{nn}/{module}|W_hat.pt" spec: weight_orig of the written
    tensor == the saved W_hat [out, in].  Returns [(spec, equal, maxabs)]."""
    import torch
    from safetensors import safe_open
    weight_map = json.loads(
        (Path(outdir) / "model.safetensors.index.json").read_text())["weight_map"]
    results = []
    for spec in what_if:
        tensor_ref, w_path = spec.split("|")
        ldir, module = tensor_ref.split("/", 1)
        base = f"{LAYER_PREFIX}{int(ldir[1:])}.{module}"
        fields = {}
        for fld in QUANT_FIELDS:            # a module's fields may sit in different shards
            with safe_open(str(Path(outdir) / weight_map[f"{base}.{fld}"]), framework="pt") as f:
                fields[fld] = f.get_tensor(f"{base}.{fld}")
        trellis, suh, svh = fields["trellis"], fields["suh"], fields["svh"]
        K = int(trellis.shape[-1]) // 16
        w = weight_orig(trellis, suh, svh, K, device=device).t().contiguous().cpu()
        W_hat = torch.load(w_path, map_location="cpu", weights_only=True)
        results.append((tensor_ref, bool(torch.equal(w, W_hat.contiguous())),
                        float((w - W_hat).abs().max())))
    return results


def check_keys(template, outdir):
    """[(key, problem)] for template keys missing from the output or with a
    different dtype/shape there."""
    template, outdir = Path(template), Path(outdir)
    t_map = json.loads((template / "model.safetensors.index.json").read_text())["weight_map"]
    o_map = json.loads((outdir / "model.safetensors.index.json").read_text())["weight_map"]
    headers: dict = {}

    def header(path):
        if path not in headers:
            headers[path] = read_st_header(path)[0]
        return headers[path]

    problems = []
    for key, shard in t_map.items():
        if key not in o_map:
            problems.append((key, "missing-from-index"))
            continue
        te = header(template / shard).get(key)
        oe = header(outdir / o_map[key]).get(key)
        if oe is None:
            problems.append((key, "missing-in-shard"))
        elif (te["dtype"], te["shape"]) != (oe["dtype"], oe["shape"]):
            problems.append((key, f"{te['dtype']}{te['shape']} vs {oe['dtype']}{oe['shape']}"))
    return problems


def _same_bytes(a: Path, b: Path) -> bool:
    if a.stat().st_size != b.stat().st_size:
        return False
    with open(a, "rb") as fa, open(b, "rb") as fb:
        while True:
            x, y = fa.read(1 << 24), fb.read(1 << 24)
            if x != y:
                return False
            if not x:
                return True


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--tensors")
    ap.add_argument("--template", required=True)
    ap.add_argument("--out", required=True)
    ap.add_argument("--selftest-a", action="store_true",
                    help="rebuild the template from its own tensors; the output shards "
                         "must be byte-identical")
    ap.add_argument("--selftest-b", nargs="*", default=None, metavar="L{nn}/{module}|W_hat.pt",
                    help="weight_orig(written tensor) == saved W_hat for each spec")
    ap.add_argument("--check-keys", action="store_true")
    ap.add_argument("--tmpdir", default=None,
                    help="scratch dir for --selftest-a (default: XTQ_TMPDIR or the parent "
                         "of --out)")
    args = ap.parse_args(argv)

    if args.selftest_a:
        parent = args.tmpdir or os.environ.get("XTQ_TMPDIR") or str(Path(args.out).parent)
        Path(parent).mkdir(parents=True, exist_ok=True)
        with tempfile.TemporaryDirectory(dir=parent) as td:
            root, n = selftest_a(args.template, td)
            print(f"selftest-a: extracted {n} module(s) -> {root}")
            export(root, args.template, args.out)
            same = True
            for shard in sorted(Path(args.out).glob("*.safetensors")):
                if not _same_bytes(shard, Path(args.template) / shard.name):
                    print(f"  DIFFERS: {shard.name}")
                    same = False
            print(f"selftest-a: shards byte-identical: {same}")
            return 0 if same else 1
    if not args.tensors:
        ap.error("--tensors is required unless --selftest-a")
    n = export(args.tensors, args.template, args.out)
    print(f"export: replaced {n} tensors -> {args.out}")
    rc = 0
    if args.selftest_b:
        for ref, eq, mx in selftest_b(args.template, args.out, args.selftest_b):
            print(f"selftest-b {ref}: equal={eq} maxabs={mx:.3e}")
            rc |= 0 if eq else 1
    if args.check_keys:
        bad = check_keys(args.template, args.out)
        print(f"check-keys: {len(bad)} problems")
        for b in bad[:20]:
            print("  ", b)
        rc |= 1 if bad else 0
    return rc


if __name__ == "__main__":
    sys.exit(main())
