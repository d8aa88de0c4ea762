"""Corrupted checkpoints against the loader's host code (safetensors header, JSON config, the
data invariants): 300 seeded corruptions of a small synthetic checkpoint (truncated files,
flipped header and config bytes, a bogus header length, flipped data bytes). Every call must
return 0 or an error code with a message - no crash, no read past a mapped file. (Run with the
library built with host AddressSanitizer, the same cases found no invalid access.)"""
import ctypes as C
import os
import random

from ckpt_synth import Synth
from mipkg import mi


def test_corrupted_checkpoints_are_refused_cleanly(tmp_path):
    L = mi.lib()
    base = str(tmp_path / "base")
    Synth(base, layers=1, H=256, QH=2, KVH=1, HD=128, I=256, V=512, mtp=True).write(split=1)
    st = [f for f in os.listdir(base) if f.endswith(".safetensors")][0]
    raw = open(os.path.join(base, st), "rb").read()
    cfg = open(os.path.join(base, "config.json"), "rb").read()
    rng = random.Random(1)
    buf = C.create_string_buffer(4096)
    refused = 0
    for it in range(300):
        d = str(tmp_path / f"c{it % 3}")
        os.makedirs(d, exist_ok=True)
        r, c = bytearray(raw), bytearray(cfg)
        kind = it % 6
        if kind == 0:
            r = r[:rng.randrange(len(r))]
        elif kind == 1:
            hl = int.from_bytes(r[:8], "little")
            for _ in range(rng.randrange(1, 8)):
                r[rng.randrange(8, 8 + hl)] = rng.randrange(256)
        elif kind == 2:
            r[:8] = rng.randrange(2**64).to_bytes(8, "little")
        elif kind == 3:
            for _ in range(rng.randrange(1, 6)):
                c[rng.randrange(len(c))] = rng.randrange(32, 127)
        elif kind == 4:
            c = c[:rng.randrange(len(c))]
        else:
            for _ in range(50):
                r[rng.randrange(len(r))] = rng.randrange(256)
        with open(os.path.join(d, st), "wb") as f:
            f.write(bytes(r))
        with open(os.path.join(d, "config.json"), "wb") as f:
            f.write(bytes(c))
        rc = L.mi_checkpoint_check(d.encode(), buf, 4096)
        desc = mi.ModelDesc()
        rc2 = L.mi_checkpoint_desc(d.encode(), 512, 4, C.byref(desc))
        assert rc in (0, -1, -2) and rc2 in (0, -1, -2), (it, kind, rc, rc2)
        if rc:
            refused += 1
            assert L.mi_last_error(), (it, kind)
    assert refused > 200
