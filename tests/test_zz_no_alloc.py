"""mi_argmax_static (no allocation: the chunk winners in the library's file-scope device
array) against mi_argmax (the caller's scratch) on the same logits: the same out_token rows,
cur_token, pos advance, step count and history, on two calls in a row, the second smaller
(fewer rows, a smaller vocabulary), so stale entries of the first call must not leak into the
second."""
import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync

pytestmark = pytest.mark.gpu


def ctrl_dev(pos, n_act):
    c = np.zeros(64, np.uint32)
    c[0], c[1] = pos, n_act
    return dev(c)


def run(entry, lg, M, V, used, pos, hist_len=8):
    ctrl = ctrl_dev(pos, M)
    hist = dev(np.zeros(hist_len, np.uint32))
    dl = dev(lg)
    print(f"{entry} M={M} V={V} used={used}", flush=True)
    if entry == "mi_argmax":
        part = empty((mi.lib().mi_argmax_groups(V) * M * 2,), np.uint32)
        mi.call("mi_argmax", ptr(ctrl), ptr(dl), ptr(part), ptr(hist), hist_len, M, V, used, stream())
    else:
        mi.call("mi_argmax_static", ptr(ctrl), ptr(dl), ptr(hist), hist_len, M, V, used, stream())
    sync()
    return host(ctrl, np.uint32).copy(), host(hist, np.uint32).copy()


def test_argmax_static_matches_argmax_on_two_calls():
    rng = np.random.default_rng(31)
    # first call: 4 rows of the 27B vocabulary, planted ties and a masked tail
    V1, M1 = 151936, 4
    lg1 = rng.uniform(-4, 4, (M1, V1)).astype(np.float32)
    lg1[0, 777] = lg1[0, 150000] = 9.0
    lg1[2, V1 - 5] = 50.0  # masked: used < V1 - 5
    used1 = V1 - 64
    # second call: fewer rows, a smaller vocabulary (fewer chunks than the first call wrote)
    V2, M2 = 4096, 2
    lg2 = rng.uniform(-4, 4, (M2, V2)).astype(np.float32)
    lg2[1, 4095] = 10.0
    for (lg, M, V, used, pos) in ((lg1, M1, V1, used1, 100), (lg2, M2, V2, V2, 7)):
        want = run("mi_argmax", lg, M, V, used, pos)
        got = run("mi_argmax_static", lg, M, V, used, pos)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
        assert list(got[0][10:10 + M]) == [O.argmax(lg[m], used) for m in range(M)]
        assert got[0][0] == pos + M and got[0][19] == 1
