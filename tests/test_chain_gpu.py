"""The layer chain launch (mi_engine_chain: per layer, o with the residual and the
post-attention norm, gate||up with SwiGLU, down with the residual and the next norm and the next
layer's q||k||v with attn_prep in ONE launch) against the launch-per-linear graph it replaces:
the same tokens, logits, control block and KV cache rows, bit for bit, over several steps from
the same state (both paths do every arithmetic operation in the same order), switching back and
forth (the chain leaves no hand-off word full); also at the 27B shape and with bf16
activations."""
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
    wgs = eng.chain(True)
    print(f"chain path ({wgs} work-groups per launch): {n} steps", flush=True)
    c_toks, c_lg, c_ctrl = run_steps(eng, pos, tok, n)
    c_k, c_v = kv_rows(eng, pos, pos + n)
    assert c_ctrl[mi.CTRL_DEBUG] == 0, hex(c_ctrl[mi.CTRL_DEBUG])
    assert c_toks == g_toks
    for a, b in zip(c_lg, g_lg):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(c_ctrl[:20], g_ctrl[:20])
    assert np.array_equal(c_k, g_k) and np.array_equal(c_v, g_v)
    # back to the graph and to the chain again: the same (no hand-off word was left full)
    eng.chain(False)
    b_toks, _, _ = run_steps(eng, pos, tok, n)
    assert b_toks == g_toks
    eng.chain(True)
    r_toks, r_lg, _ = run_steps(eng, pos, tok, n)
    assert r_toks == g_toks
    for a, b in zip(r_lg, g_lg):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("qk_norm,head_dim,layers,act", [(1, 128, 2, 0), (0, 128, 3, 0), (1, 256, 2, 0),
                                                          (1, 128, 1, 0), (1, 128, 2, 1)])
def test_chain_bitwise_graph_small(qk_norm, head_dim, layers, act):
    """layers 1 and 3: the launch that empties the last layer's words runs in every step."""
    eng = mi.Engine(small_desc(qk_norm=qk_norm, head_dim=head_dim, layers=layers, max_len=512, act_bf16=act),
                    seed=21)
    compare_paths(eng, 300, 7, 4)
    eng.close()


def test_chain_verify_rows_bitwise_chain_steps():
    """verify keeps the graph of launches (rows > 1); its rows are bitwise the chain's steps."""
    eng = mi.Engine(small_desc(max_rows=4), seed=8)
    eng.capture(1)
    eng.chain(True)
    P, t0 = 40, 3
    eng.reset(P, t0)
    toks, lg = [], []
    for _ in range(4):
        toks.append(int(eng.generate(1)[0]))
        lg.append(eng.logits(1)[0].copy())
    eng.reset(P, t0)
    rows = eng.verify(toks[:3])
    assert list(rows) == toks
    got = eng.logits(4)
    for m in range(4):
        assert np.array_equal(got[m].view(np.uint32), lg[m].view(np.uint32))
    eng.close()


def test_chain_refusals():
    with pytest.raises(mi.MiError):
        eng = mi.Engine(small_desc(kv_int8=1, head_dim=256), seed=1)
        try:
            eng.chain(True)
        finally:
            eng.close()


def test_chain_bitwise_graph_27b():
    print("building the 27B-shape engine", flush=True)
    eng = mi.Engine(mi.desc_27b(max_len=4160), seed=1234)
    compare_paths(eng, 4096, 1000, 3)
    eng.close()
