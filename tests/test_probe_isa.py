"""The VALU issue-rate probe counts what it issues.

bench.py turns each probe's time into lane-instructions per second with the
per-chain instruction counts in probe/valu_probe.hip (kOpsPerChain).  This
test compiles the probe for gfx950 to device assembly (hipcc, no GPU needed)
and checks, for every probe index, that the timed loop issues exactly those
instructions: per loop iteration (the compiler's unroll factor read from the
loop counter's step), kChains times the probe's per-chain opcode mix and no
other vector instruction -- except the two packed-fp16-codebook mixes, which
carry four integer operations of loop overhead per iteration (6 % of their
VALU instructions; not counted as work, so their rates are slight
underestimates).  A probe whose loop lost or gained an instruction would
state a wrong ceiling.
"""
import collections
import os
import re
import shutil
import subprocess

import pytest

from conftest import PKG

SRC = os.path.join(PKG, "probe", "valu_probe.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# probe index -> (kernel template arguments, per-chain opcode mix)
FP32_MIX = {"v_add_f32": 2, "v_mul_f32": 1, "v_min_f64": 1}
MIN_ONLY_MIX = {"v_add_f32": 2, "v_mul_f32": 1}          # plus the min3 tree per 8 chains
FP16_MIX = {"v_fma_mix_f32": 1, "v_mul_f32": 1, "v_add_f32": 1, "v_min_f64": 1}
PROBES = {
    0: ("0, false", {"v_mul_f32": 1}),
    1: ("1, false", {"v_add_f32": 1}),
    2: ("2, false", {"v_fma_f32": 1}),
    3: ("3, false", {"v_fma_mix_f32": 1}),
    4: ("4, false", {"v_min_f64": 1}),
    5: ("5, false", FP16_MIX),
    6: ("6, false", FP16_MIX),
    7: ("7, false", FP32_MIX),
    8: ("8, false", FP32_MIX),
    9: ("9, false", {"v_min3_f32": 1}),
    10: ("10, false", MIN_ONLY_MIX),
    11: ("8, true", FP32_MIX),
    12: ("10, true", MIN_ONLY_MIX),
}


def _source_constants():
    text = open(SRC).read()
    chains = int(re.search(r"constexpr int kChains = (\d+);", text).group(1))
    ops = re.search(r"constexpr double kOpsPerChain\[(\d+)\] = \{([^}]*)\};", text)
    vals = [float(v) for v in ops.group(2).split(",")]
    assert int(ops.group(1)) == len(vals)
    return chains, vals


@pytest.fixture(scope="module")
def loops(tmp_path_factory):
    if not os.path.exists(HIPCC) and not shutil.which("hipcc"):
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("probe_isa") / "valu_probe.s")
    subprocess.run([HIPCC if os.path.exists(HIPCC) else "hipcc", "--offload-arch=gfx950", "-O3",
                    "-std=c++17", "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                    "--cuda-device-only", "-S", SRC, "-o", out],
                   check=True, capture_output=True)
    text = open(out).read()
    found = {}
    for m in re.finditer(r"^(_Z\S*probe_kernel\S*):[^\n]*\n(.*?)^\s*s_endpgm", text, re.S | re.M):
        name = subprocess.run(["c++filt", m.group(1)], capture_output=True, text=True,
                              check=True).stdout
        args = re.search(r"probe_kernel<([^>]*)>", name).group(1)
        lines = [ln for ln in m.group(2).split("\n") if "ASM" not in ln]
        labels = {ln.split(":")[0]: i for i, ln in enumerate(lines)
                  if re.match(r"^\.LBB\d+_\d+:", ln)}
        back = [(labels[b.group(1)], i) for i, ln in enumerate(lines)
                for b in [re.match(r"\s*s_cbranch_\w+\s+(\.LBB\d+_\d+)", ln)]
                if b and b.group(1) in labels and labels[b.group(1)] < i]
        assert len(back) == 1, (args, "one timed loop")
        body = lines[back[0][0]:back[0][1] + 1]
        step = [int(s.group(1)) for ln in body
                for s in [re.match(r"\s*s_add_i32 s\d+, s\d+, -(\d+)$", ln)] if s]
        assert len(step) == 1, (args, body)
        valu = collections.Counter(re.match(r"\s+(v_\w+)", ln).group(1).replace("_e32", "")
                                   .replace("_e64", "") for ln in body if re.match(r"\s+v_", ln))
        found[args] = (step[0], valu)
    return found


@pytest.mark.parametrize("which", sorted(PROBES))
def test_probe_loop_issues_its_counted_instructions(loops, which):
    chains, ops_per_chain = _source_constants()
    args, mix = PROBES[which]
    unroll, valu = loops[args]
    per_iter = {op: n / unroll for op, n in valu.items()}
    probed = {op: per_iter.get(op, 0) for op in mix}
    if which in (10, 12):
        # add, mul, add per chain and a v_min3_f32 tree over each 8 chains
        # (three v_min3_f32 and one v_min_f32)
        probed.update(v_min3_f32=per_iter.get("v_min3_f32", 0),
                      v_min_f32=per_iter.get("v_min_f32", 0))
        want = {op: n * chains for op, n in mix.items()}
        want.update(v_min3_f32=3 * chains / 8, v_min_f32=chains / 8)
    else:
        want = {op: n * chains for op, n in mix.items()}
    assert probed == want, (which, per_iter)
    work = sum(want.values())
    assert work == chains * ops_per_chain[which], (which, work)
    other = sum(per_iter.values()) - work
    assert other == 0 or (which in (5, 6) and other <= 4), (which, per_iter)
