"""Properties of the generated gfx950 code that the decode kernels' correctness relies on.

The slab and head decode kernels hand the q/k conv history of a (sequence, q/k head) group
to the group's last member through a relaxed atomic counter (baloon_amd/csrc/gdn_decode.hip,
file header). One of the facts that hand-off rests on is about code generation, not the HIP
memory model: the global atomic add must come after the workgroup's s_barrier, which follows
every member's conv-history reads. This test compiles gdn_decode.hip to AMD assembly with
the library's own flags and checks that order in every slab and head kernel. No GPU needed.
"""
import os
import re
import subprocess
import tempfile

import pytest

from baloon_amd import build as b

SRC = os.path.join(b.CSRC, "gdn_decode.hip")


@pytest.fixture(scope="module")
def decode_asm():
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "decode.s")
        cmd = [b.HIPCC, *b.FLAGS, *b.FILE_FLAGS.get("gdn_decode.hip", []), "--cuda-device-only", "-S", SRC, "-o", out]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
        assert r.returncode == 0, r.stderr
        return open(out).read()


def kernel_bodies(asm: str):
    """{mangled name: body text} of every kernel function in the assembly."""
    heads = list(re.finditer(r"^(_Z\S+):\s*;\s*@", asm, re.M))
    out = {}
    for i, m in enumerate(heads):
        end = heads[i + 1].start() if i + 1 < len(heads) else len(asm)
        body = asm[m.end():end]
        stop = body.find("s_endpgm")
        out[m.group(1)] = body if stop < 0 else body[:stop]
    return out


def test_counter_atomic_follows_the_barrier(decode_asm):
    bodies = kernel_bodies(decode_asm)
    checked = 0
    for name, body in bodies.items():
        if "slab_kernel" not in name and "head_kernel" not in name:
            continue
        atomic = body.find("global_atomic_add")
        barrier = body.find("s_barrier")
        assert atomic >= 0, f"{name}: no counter atomic found"
        assert 0 <= barrier < atomic, f"{name}: the counter atomic precedes the first s_barrier"
        checked += 1
    # slab kernels: 3 conv widths x 2 group sizes; head kernels: 3 conv widths
    assert checked == 9, sorted(bodies)
