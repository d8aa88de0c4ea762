"""The persistent one-launch decode step (mi_engine_persistent) against the captured graph of
launches it replaces: the same tokens, logits, control block and KV cache rows, bit for bit, over
several steps from the same state (both paths do every arithmetic operation in the same order);
and the 27B-shape step the same way."""
import numpy as np
import pytest

from mipkg import mi
from test_engine_gpu import small_desc

pytestmark = pytest.mark.gpu


def run_steps(eng, pos, tok, n):
    eng.reset(pos, tok)
    toks, lg = [], []
    for _ in range(n):
        toks.append(int(eng.generate(1)[0]))
        lg.append(eng.logits(1)[0].copy())
    return toks, lg, eng.ctrl().copy()


def kv_rows(eng, lo, hi):
    d = eng.desc
    shp = (d.layers, d.kv_heads, d.max_len, d.head_dim)
    k = eng.to_host(mi.T_KV_K, 0, np.uint16).reshape(shp)[:, :, lo:hi].copy()
    v = eng.to_host(mi.T_KV_V, 0, np.uint16).reshape(shp)[:, :, lo:hi].copy()
    return k, v


def compare_paths(eng, pos, tok, n):
    eng.capture(1)
    print(f"graph path: {n} steps from pos {pos}", flush=True)
    g_toks, g_lg, g_ctrl = run_steps(eng, pos, tok, n)
    g_k, g_v = kv_rows(eng, pos, pos + n)
    wgs = eng.persistent(True)
    print(f"persistent path ({wgs} work-groups): {n} steps", flush=True)
    p_toks, p_lg, p_ctrl = run_steps(eng, pos, tok, n)
    p_k, p_v = kv_rows(eng, pos, pos + n)
    assert p_ctrl[mi.CTRL_DEBUG] == 0, hex(p_ctrl[mi.CTRL_DEBUG])
    assert p_toks == g_toks
    for a, b in zip(p_lg, g_lg):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(p_ctrl[:20], g_ctrl[:20])
    assert np.array_equal(p_k, g_k) and np.array_equal(p_v, g_v)
    # and back to the graph: the same again (the persistent step left no hand-off word full)
    eng.persistent(False)
    b_toks, b_lg, _ = run_steps(eng, pos, tok, n)
    assert b_toks == g_toks
    eng.persistent(True)
    r_toks, r_lg, _ = run_steps(eng, pos, tok, n)
    assert r_toks == g_toks
    for a, b in zip(r_lg, g_lg):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("qk_norm,head_dim", [(1, 128), (0, 128), (1, 256)])
def test_persistent_step_bitwise_graph_small(qk_norm, head_dim):
    eng = mi.Engine(small_desc(qk_norm=qk_norm, head_dim=head_dim, max_len=512), seed=21)
    compare_paths(eng, 300, 7, 4)
    eng.close()


def test_persistent_step_bitwise_graph_27b():
    eng = mi.Engine(mi.desc_27b(max_len=4160), seed=1234)
    compare_paths(eng, 4096, 1000, 3)
    eng.close()
