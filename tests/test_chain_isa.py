"""The column-chain kernel publishes tiles the way its memory-ordering
argument assumes.

ldlq_chain_kernel<K> writes each tile's error E with agent-scope stores and
stores the tile's flag once every wave's stores have completed, without the
L2 write-back (buffer_wbl2) of an agent-scope release; the waiter's acquire
fence invalidates its L2 before it reads E.  This test compiles the kernels
for gfx950 to device assembly (hipcc, no GPU needed) and checks, for every K,
that the chain kernel issues no buffer_wbl2, that its E and flag stores are
agent-scope (sc1) stores, that a vmcnt(0) wait precedes the barrier before the
flag store, and that the acquire's buffer_inv sc1 is there.  A compiler that
emitted a relaxed agent-scope store without sc1 (or a plain store for E) would
break the publication silently; this catches it at build time.
"""
import os
import re
import shutil
import subprocess

import pytest

from conftest import PKG

SRC = os.path.join(PKG, "csrc", "viterbi_kernels.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.fixture(scope="module")
def chain_bodies(tmp_path_factory):
    if not os.path.exists(HIPCC) and not shutil.which("hipcc"):
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("chain_isa") / "viterbi_kernels.s")
    subprocess.run([HIPCC if os.path.exists(HIPCC) else "hipcc", "--offload-arch=gfx950", "-O3",
                    "-std=c++17", "-ffp-contract=off", "-fvisibility=hidden",
                    "-fno-gpu-flush-denormals-to-zero",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                    "--cuda-device-only", "-S", SRC, "-o", out],
                   check=True, capture_output=True)
    text = open(out).read()
    bodies = {}
    for m in re.finditer(r"^(_Z\S*ldlq_chain_kernelILi(\d)E\S*):[^\n]*\n(.*?)^\s*s_endpgm",
                         text, re.S | re.M):
        bodies[int(m.group(2))] = m.group(3)
    return bodies


@pytest.mark.parametrize("K", [2, 3, 4, 5, 6, 7])
def test_chain_publish_without_l2_writeback(chain_bodies, K):
    body = chain_bodies[K]
    lines = [ln.strip() for ln in body.split("\n")]
    assert not any(ln.startswith("buffer_wbl2") for ln in lines), "an L2 write-back in the loop"
    # the waiter's acquire: one L2 invalidate after its flag poll
    assert sum(ln.startswith("buffer_inv sc1") for ln in lines) >= 1
    # E (256 threads) and the flag (thread 0): agent-scope global stores
    sc1_stores = [i for i, ln in enumerate(lines)
                  if re.match(r"global_store_dword\s.*\bsc1\b", ln)]
    assert len(sc1_stores) >= 2, "E and flag stores must be agent-scope (sc1)"
    # the flag store is the last sc1 store; before it: vmcnt(0), then the barrier
    flag = sc1_stores[-1]
    bar = max(i for i in range(flag) if lines[i] == "s_barrier")
    assert any("s_waitcnt vmcnt(0)" in lines[i] for i in range(bar - 4, bar)), \
        "every wave waits for its stores before the barrier that precedes the flag"
