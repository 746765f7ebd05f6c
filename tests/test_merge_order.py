"""The order in which the split Q4_K products' parts meet, checked in the
gfx950 assembly of this build's own kernels (k_mv_q4k_mfma.hip, one token;
k_mv_q4k_stream.hip, two to four tokens).

The parts of a tile are summed by the last workgroup to count in.  Without a
release/acquire fence (whose cache maintenance would write back or drop the
XCD's L2), the ordering rests on this sequence, which the test asserts for
every counter add of every kernel:
  * the partial sums are stored device-coherently (`global_store ... sc1`);
  * an `s_waitcnt` with `vmcnt(0)` lies between the last such store and the counter's
    `global_atomic_add ... sc0` (the add with its old value returned);
  * after the add, such a wait and a branch on its result come
    before the first device-coherent load of the partial sums
    (`global_load ... sc1`).
Compiles with hipcc (no GPU needed).
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "dwim_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _kernels(src, tmp_path):
    out = tmp_path / (src + ".s")
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-Wno-unused-command-line-argument", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    kernels, name = {}, None
    for line in out.read_text().splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            name = m.group(1)
            kernels[name] = []
        elif name:
            kernels[name].append(line.strip())
    return kernels


def _check_meetings(body):
    adds = [i for i, l in enumerate(body) if l.startswith("global_atomic_add") and l.endswith("sc0")]
    for i in adds:
        stores = [j for j in range(i) if l_is(body[j], "global_store") and "sc1" in body[j].split()]
        assert stores, "no device-coherent partial store before the counter add"
        assert any(_vm0(l) for l in body[stores[-1] + 1:i]), "the add may issue before the stores complete"
        loads = [j for j in range(i + 1, len(body)) if l_is(body[j], "global_load") and "sc1" in body[j].split()]
        assert loads, "no device-coherent partial load after the counter add"
        between = body[i + 1:loads[0]]
        w = next((k for k, l in enumerate(between) if _vm0(l)), None)
        assert w is not None, "the partial loads may issue before the add returns"
        assert any(l.startswith("s_cbranch") for l in between[w:]), "no branch on the add's result"
    return len(adds)


def _vm0(line):
    """An s_waitcnt that waits for every vector memory operation (vmcnt(0),
    alone or with other counters)."""
    return line.startswith("s_waitcnt") and "vmcnt(0)" in line.split()


def l_is(line, op):
    return line.startswith(op)


@pytest.mark.parametrize("src,kernel", [("k_mv_q4k_mfma.hip", "k_mv_q4k_mfma"), ("k_mv_q4k_stream.hip", "k_mv_stream")])
def test_parts_meet_after_their_stores_complete(src, kernel, tmp_path):
    kernels = {k: v for k, v in _kernels(src, tmp_path).items() if kernel in k}
    assert kernels
    checked = sum(_check_meetings(body) for body in kernels.values())
    assert checked >= len(kernels)
