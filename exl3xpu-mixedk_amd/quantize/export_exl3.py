#!/usr/bin/env python3
"""export_exl3.py -- put trellis-quantized tensors into an EXL3 model directory.

Drop-in for the reference's writer (quantize/export_exl3.py): the same
functions, command line, input layout and exceptions.

Input layout (--tensors ROOT), one file per quantized module:

    ROOT/L{nn}/{module}.safetensors   trellis int16 [k/16, n/16, 16K],
                                      suh fp16 [k], svh fp16 [n]
    ROOT/L{nn}/{module}.json          optional metadata; its "module" names the
                                      module when the file stem does not

A module's tensors land on model.language_model.layers.{nn}.{module}.{field}
of the template (--template, an EXL3 model directory: index + shards).

How the output (--out) is made: every input is validated against the
template's shard headers first (key present, dtype, shape, byte size); only
then is anything written.  Shards are copied with the provided tensors'
bytes overwritten where the template stores them, so headers never change
and writing a template's own tensors back reproduces its shards byte for
byte.  Other files are copied as they are and ARTIFACTS.sha256 is rebuilt
over the output.

Checks: --selftest-a extracts the template's own decoder-layer tensors into
the input layout and rebuilds the template from them (shards must be
byte-identical); --selftest-b reconstructs written tensors with a decoder
independent of the GPU kernels (torch integer ops on the bit stream, then
the inverse incoherence transform) and compares them with a saved W_hat;
--check-keys lists template keys missing from the output or stored there
with another dtype or shape.

write_quantized() is the quantizer side: it stores one quantize_linear
result in the input layout.  weight_orig() is the GPU reconstruction (HIP
decode) the quantizer itself uses.
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

QUANT_FIELDS = ("trellis", "suh", "svh")
LAYER_PREFIX = "model.language_model.layers."
INDEX_NAME = "model.safetensors.index.json"
ARTIFACTS = "ARTIFACTS.sha256"

# safetensors dtype tag -> torch dtype name, for the tags an input may carry
_TAG_TO_TORCH = {"I16": "int16", "F16": "float16", "F32": "float32", "I32": "int32",
                 "I64": "int64", "U8": "uint8", "BOOL": "bool", "BF16": "bfloat16"}
_INPUT_TAGS = frozenset(("I16", "F16", "F32", "I32", "I64", "U8", "BOOL"))


# ------------------------------------------------------------ safetensors
class _StFile:
    """A safetensors file's header: tensor name -> (dtype tag, shape, absolute
    first byte, absolute end byte).  The format is an 8-byte little-endian
    header length, a JSON header with per-tensor data_offsets relative to the
    data section, then the data section."""

    def __init__(self, path):
        self.path = Path(path)
        with open(self.path, "rb") as f:
            (hlen,) = struct.unpack("<Q", f.read(8))
            self.header = json.loads(f.read(hlen))
        self.data_start = 8 + hlen
        self.entries = {}
        for name, ent in self.header.items():
            if name == "__metadata__":
                continue
            lo, hi = ent["data_offsets"]
            self.entries[name] = (ent["dtype"], list(ent["shape"]), self.data_start + lo,
                                  self.data_start + hi)

    def read(self, name: str) -> bytes:
        _, _, a, b = self.entries[name]
        with open(self.path, "rb") as f:
            f.seek(a)
            return f.read(b - a)

    def tensor(self, name: str):
        """The tensor as a torch tensor (CPU, a copy)."""
        import torch
        tag, shape, _, _ = self.entries[name]
        dtype = getattr(torch, _TAG_TO_TORCH[tag])
        return torch.frombuffer(bytearray(self.read(name)), dtype=dtype).reshape(shape).clone()


def read_st_header(path):
    """(header dict, byte offset of the data section) of a safetensors file."""
    f = _StFile(path)
    return f.header, f.data_start


def tensor_bytes(path, key):
    """Raw bytes of tensor `key` inside safetensors file `path`."""
    return _StFile(path).read(key)


def _weight_map(model_dir) -> dict:
    return json.loads((Path(model_dir) / INDEX_NAME).read_text())["weight_map"]


def _split_layer_key(key: str):
    """'model.language_model.layers.{nn}.{module}.{field}' -> (nn, module,
    field), or None for keys outside the decoder layers."""
    if not key.startswith(LAYER_PREFIX):
        return None
    nn, _, rest = key[len(LAYER_PREFIX):].partition(".")
    module, _, field = rest.rpartition(".")
    return int(nn), module, field


# ------------------------------------------------------------------ inputs
def _input_files(tensors_root):
    """(layer, module, path) of every input file, in path order."""
    for path in sorted(Path(tensors_root).glob("L*/*.safetensors")):
        module = path.stem
        meta = path.with_suffix(".json")
        if meta.exists():
            module = json.loads(meta.read_text()).get("module", module)
        yield int(path.parent.name[1:]), module, path


def collect_inputs(tensors_root):
    """Every quantized tensor under ROOT/L*/ -> {template key: (dtype tag,
    shape, raw bytes)}.  A file without one of trellis/suh/svh raises
    KeyError; a dtype the template cannot hold raises ValueError."""
    found = {}
    for layer, module, path in _input_files(tensors_root):
        st = _StFile(path)
        for field in QUANT_FIELDS:
            if field not in st.entries:
                raise KeyError(f"{path}: no {field!r} tensor (it holds "
                               f"{sorted(st.entries)})")
        for field in QUANT_FIELDS:
            tag, shape, _, _ = st.entries[field]
            if tag not in _INPUT_TAGS:
                raise ValueError(f"{path}:{field} has dtype {tag}, which the writer "
                                 "does not take")
            found[f"{LAYER_PREFIX}{layer}.{module}.{field}"] = (tag, shape, st.read(field))
    return found


def write_quantized(root, layer: int, module: str, result: dict, extra_meta=None) -> Path:
    """Store one quantize_linear result (trellis, suh, svh) as
    ROOT/L{layer:02d}/{module}.safetensors plus its .json metadata."""
    import torch
    from safetensors.torch import save_file
    path = Path(root) / f"L{int(layer):02d}" / f"{module}.safetensors"
    path.parent.mkdir(parents=True, exist_ok=True)
    want = {"trellis": torch.int16, "suh": torch.float16, "svh": torch.float16}
    save_file({f: result[f].to("cpu", dt).contiguous() for f, dt in want.items()}, str(path))
    meta = {"module": module, "K": int(result.get("K", result["trellis"].shape[-1] // 16))}
    meta.update({k: result[k] for k in ("Wscale", "code", "channel_scales", "use_ldlq")
                 if k in result})
    meta.update(extra_meta or {})
    path.with_suffix(".json").write_text(json.dumps(meta))
    return path


# ------------------------------------------------------------------ export
def _plan(inputs: dict, template: Path, weight_map: dict) -> dict:
    """Validate every input against the template before any write: shard
    name -> [(absolute offset, raw bytes, key)]."""
    by_shard: dict = {}
    for key in sorted(inputs):
        shard = weight_map.get(key)
        if shard is None:
            raise KeyError(f"input key {key} is not in the template's index")
        by_shard.setdefault(shard, []).append(key)
    plan = {}
    for shard, keys in by_shard.items():
        st = _StFile(template / shard)
        writes = []
        for key in keys:
            tag, shape, raw = inputs[key]
            if key not in st.entries:
                raise KeyError(f"input key {key} is not in template shard {shard}")
            t_tag, t_shape, a, b = st.entries[key]
            if tag != t_tag:
                raise ValueError(f"{key}: dtype {tag} where the template has {t_tag}")
            if shape != t_shape:
                raise ValueError(f"{key}: shape {shape} where the template has {t_shape}")
            if len(raw) != b - a:
                raise ValueError(f"{key}: {len(raw)} bytes where the template has {b - a}")
            writes.append((a, raw, key))
        plan[shard] = writes
    return plan


def _sha256_file(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 24), b""):
            h.update(block)
    return h.hexdigest()


def _write_artifacts(outdir: Path):
    """ARTIFACTS.sha256 over the output files, in sha256sum's format."""
    names = sorted(p.name for p in outdir.iterdir() if p.is_file() and p.name != ARTIFACTS)
    (outdir / ARTIFACTS).write_text(
        "".join(f"{_sha256_file(outdir / n)}  {n}\n" for n in names))


def export(tensors_root, template, outdir):
    """Splice the quantized tensors under tensors_root into a copy of the
    template directory; returns the number of tensors written."""
    template, outdir = Path(template), Path(outdir)
    weight_map = _weight_map(template)
    inputs = collect_inputs(tensors_root)
    plan = _plan(inputs, template, weight_map)
    shards = set(weight_map.values())
    outdir.mkdir(parents=True, exist_ok=True)
    written = 0
    for shard in sorted(shards):
        shutil.copyfile(template / shard, outdir / shard)
        writes = plan.get(shard, ())
        if writes:
            with open(outdir / shard, "r+b") as f:
                for offset, raw, _ in writes:
                    f.seek(offset)
                    f.write(raw)
            written += len(writes)
    if written != len(inputs):
        raise RuntimeError(f"{len(inputs) - written} input tensors were not written")
    for item in template.iterdir():
        if item.is_file() and item.name not in shards and item.name != ARTIFACTS:
            shutil.copyfile(item, outdir / item.name)
    _write_artifacts(outdir)
    return written


# ------------------------------------------------------------------ checks
def selftest_a(template, workdir, only_keys=None):
    """The template's own decoder-layer quantized tensors in the input layout
    under workdir/tensors; returns (root, files written).  Keys outside
    model.language_model.layers.* (lm_head, mtp.*) have no input layout and
    keep the template bytes."""
    from safetensors.torch import save_file
    template = Path(template)
    modules: dict = {}
    shard_keys: dict = {}
    for key, shard in _weight_map(template).items():
        parts = _split_layer_key(key)
        if parts is None or parts[2] not in QUANT_FIELDS:
            continue
        if only_keys is None or key in only_keys:
            shard_keys.setdefault(shard, []).append((key, parts))
    for shard, items in shard_keys.items():
        st = _StFile(template / shard)
        for key, (layer, module, field) in items:
            modules.setdefault((layer, module), {})[field] = st.tensor(key)
    root = Path(workdir) / "tensors"
    for (layer, module), tensors in sorted(modules.items()):
        path = root / f"L{layer}" / f"{module}.safetensors"
        path.parent.mkdir(parents=True, exist_ok=True)
        save_file(tensors, str(path))
        K = int(tensors["trellis"].shape[-1]) // 16 if "trellis" in tensors else 4
        path.with_suffix(".json").write_text(json.dumps({"module": module, "K": K}))
    return root, len(modules)


def weight_orig(trellis, suh, svh, K: int, code: str = "exl3_mul1", device=None):
    """Original-basis weight [k, n] fp32 of one EXL3 tensor: the HIP trellis
    decode, then diag(suh) B W_inner B diag(svh) (the inverse incoherence
    transform, quantize.py:158-164).  quantize_linear builds W_hat with the
    same operations, so W_hat == weight_orig(...).t() on the same device."""
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import hip_backend as hb
    import quantize as xq
    dev = torch.device(device) if device is not None else torch.device("cuda")
    w_inner = hb.decode(trellis.to("cuda", torch.int16).contiguous(), int(K),
                        code=hb.code_name(code)).to(dev)
    return xq.from_inner(w_inner, suh.to(dev), svh.to(dev), xq.hadamard128(dev, torch.float32))


def _states_from_stream(trellis, K: int):
    """int16 [tiles, 16K] -> int64 states [tiles, 256] with torch integer ops
    (no GPU kernel): the stream's 32-bit words are (lo16 | hi16 << 16), bit b
    of the stream is bit 31 - b%32 of word b/32, and s_t is the 16 stream
    bits ending at bit (t+1)K - 1, read circularly, MSB first
    (quantize.py:381-402)."""
    import torch
    t16 = trellis.to(torch.int64) & 0xFFFF
    words = t16[:, 0::2] | (t16[:, 1::2] << 16)                   # [tiles, 8K]
    nbits = 256 * K
    b = torch.arange(nbits, device=trellis.device)
    bits = (words[:, b // 32] >> (31 - b % 32)) & 1                 # [tiles, 256K]
    t = torch.arange(256, device=trellis.device).unsqueeze(1)
    k = torch.arange(16, device=trellis.device).unsqueeze(0)
    idx = (t * K + K - 16 + k) % nbits                              # [256, 16]
    weights = (1 << (15 - torch.arange(16, device=trellis.device)))
    return (bits[:, idx] * weights).sum(dim=2)


def weight_orig_torch(trellis, suh, svh, K: int, code: str = "exl3_mul1", device=None,
                      tiles_per_block: int = 4096):
    """weight_orig through a decoder independent of the GPU kernels: the bit
    stream is unpacked with torch integer ops (_states_from_stream), mapped
    through the codebook table and placed by the tensor-core permutation
    (quantize.py:101-118,405-415), then taken through the same inverse
    incoherence transform.  The check --selftest-b runs."""
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import quantize as xq
    dev = torch.device(device) if device is not None else torch.device("cuda")
    tk, tn, w = trellis.shape
    if w != 16 * K:
        raise ValueError(f"trellis last dim {w} != 16 K = {16 * K}")
    lut = xq.get_lut(code).to(dev, torch.float32)
    perm = xq.tensor_core_perm().to(dev)
    flat = trellis.to(dev).reshape(tk * tn, w)
    tiles = torch.empty(tk * tn, 256, dtype=torch.float32, device=dev)
    for a in range(0, tk * tn, tiles_per_block):
        st = _states_from_stream(flat[a:a + tiles_per_block], K)
        tiles[a:a + tiles_per_block, perm] = lut[st]
    w_inner = tiles.view(tk, tn, 16, 16).permute(0, 2, 1, 3).reshape(16 * tk, 16 * tn)
    return xq.from_inner(w_inner, suh.to(dev), svh.to(dev), xq.hadamard128(dev, torch.float32))


def _module_fields(model_dir: Path, weight_map: dict, base: str) -> dict:
    """trellis/suh/svh of one module, wherever the index puts each field."""
    return {f: _StFile(model_dir / weight_map[f"{base}.{f}"]).tensor(f"{base}.{f}")
            for f in QUANT_FIELDS}


def selftest_b(template, outdir, what_if, device=None):
    """For each "L{nn}/{module}|W_hat.pt" spec: the written tensor,
    reconstructed by weight_orig_torch (a decoder independent of the
    quantizer's), equals the saved W_hat [out, in].  Returns
    [(spec tensor, equal, max abs difference)]."""
    import torch
    outdir = Path(outdir)
    weight_map = _weight_map(outdir)
    results = []
    for spec in what_if:
        tensor_ref, w_path = spec.split("|")
        ldir, module = tensor_ref.split("/", 1)
        fields = _module_fields(outdir, weight_map, f"{LAYER_PREFIX}{int(ldir[1:])}.{module}")
        K = int(fields["trellis"].shape[-1]) // 16
        w = weight_orig_torch(fields["trellis"], fields["suh"], fields["svh"], K,
                              device=device).t().contiguous().cpu()
        W_hat = torch.load(w_path, map_location="cpu", weights_only=True).contiguous()
        results.append((tensor_ref, bool(torch.equal(w, W_hat)),
                        float((w - W_hat).abs().max())))
    return results


def check_keys(template, outdir):
    """[(key, problem)] for template keys missing from the output's index or
    shard, or stored there with another dtype or shape."""
    template, outdir = Path(template), Path(outdir)
    t_map, o_map = _weight_map(template), _weight_map(outdir)
    opened: dict = {}

    def entries(path: Path):
        if path not in opened:
            opened[path] = _StFile(path).entries
        return opened[path]

    problems = []
    for key, shard in t_map.items():
        if key not in o_map:
            problems.append((key, "missing-from-index"))
            continue
        o_ent = entries(outdir / o_map[key]).get(key)
        if o_ent is None:
            problems.append((key, "missing-in-shard"))
            continue
        t_tag, t_shape = entries(template / shard)[key][:2]
        if (t_tag, t_shape) != o_ent[:2]:
            problems.append((key, f"{t_tag}{t_shape} vs {o_ent[0]}{o_ent[1]}"))
    return problems


def _files_equal(a: Path, b: Path) -> bool:
    return a.stat().st_size == b.stat().st_size and _sha256_file(a) == _sha256_file(b)


def main(argv=None):
    ap = argparse.ArgumentParser(description="Write trellis-quantized tensors into an EXL3 "
                                             "model directory.")
    ap.add_argument("--tensors", help="input root: L{nn}/{module}.safetensors (+ .json)")
    ap.add_argument("--template", required=True, help="EXL3 model directory to start from")
    ap.add_argument("--out", required=True, help="output model directory")
    ap.add_argument("--selftest-a", action="store_true",
                    help="rebuild the template from its own tensors and require "
                         "byte-identical shards")
    ap.add_argument("--selftest-b", nargs="*", default=None, metavar="L{nn}/{module}|W_hat.pt",
                    help="reconstruct each written tensor independently and require it "
                         "to equal the saved W_hat")
    ap.add_argument("--check-keys", action="store_true",
                    help="list template keys missing from the output or changed in "
                         "dtype/shape")
    ap.add_argument("--tmpdir", default=None,
                    help="where --selftest-a extracts (default: XTQ_TMPDIR, else the "
                         "directory holding --out)")
    args = ap.parse_args(argv)

    if args.selftest_a:
        scratch = Path(args.tmpdir or os.environ.get("XTQ_TMPDIR") or Path(args.out).parent)
        scratch.mkdir(parents=True, exist_ok=True)
        with tempfile.TemporaryDirectory(dir=scratch) as td:
            root, n = selftest_a(args.template, td)
            print(f"selftest-a: {n} module(s) extracted to {root}")
            export(root, args.template, args.out)
            differ = [p.name for p in sorted(Path(args.out).glob("*.safetensors"))
                      if not _files_equal(p, Path(args.template) / p.name)]
            for name in differ:
                print(f"  DIFFERS: {name}")
            print(f"selftest-a: shards byte-identical: {not differ}")
            return 1 if differ else 0
    if not args.tensors:
        ap.error("--tensors is required unless --selftest-a is given")
    n = export(args.tensors, args.template, args.out)
    print(f"export: {n} tensors written to {args.out}")
    rc = 0
    if args.selftest_b:
        for ref, eq, mx in selftest_b(args.template, args.out, args.selftest_b):
            print(f"selftest-b {ref}: equal={eq} max|diff|={mx:.3e}")
            rc |= 0 if eq else 1
    if args.check_keys:
        bad = check_keys(args.template, args.out)
        print(f"check-keys: {len(bad)} problem(s)")
        for b in bad[:20]:
            print("  ", b)
        rc |= 1 if bad else 0
    return rc


if __name__ == "__main__":
    sys.exit(main())
