"""BASELINE's configurations at their full sizes, on the GPU, against the oracle.

- the 27B-shape dense step (64 layers, hidden 5120, 40/8 heads of 128, SwiGLU
  17408, vocab 151936, context 4096): one captured step's logits within rel 2e-3 of the
  oracle's whole step over the same weights, KV and token, argmax equal (or an oracle near-tie);
  verify at 4 and 8 rows with every row bitwise the plain step at its position, and
  accept_greedy / commit on the result.
- the small-M GEMV at the 27B shapes (5120 -> 34816 gate||up, 17408 -> 5120 down,
  5120 -> 7168 qkv) at M = 4, 8, 16: every output within the N2 bound of the fp64 product
  (tests/kernels/gemm_sm_ref.h:180-225) and within rel 2e-3 of the reference's fp32 twin;
  property R at the engine's split width (each row bitwise its 1-row launch).
- configs[2] at 131072 keys: int8 KV with fp16 scales, 64-token pages in a shuffled table:
  paged bitwise the contiguous cache, and within rel 2e-3 / cosine 0.99999 of fp64 softmax
  attention on one q head per kv head."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync
from test_attn_gpu import check_close, gpu_attention
from test_engine_gpu import OracleModel, argmax_ok, close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng27():
    print("building the 27B-shape engine (64 layers)", flush=True)
    e = mi.Engine(mi.desc_27b(max_len=4160), seed=1234)
    e.capture(1)
    yield e
    e.close()


def test_cfg2_full_27b_step_vs_oracle(eng27):
    pos, tok = 4096, 1000
    print("27B: oracle copies of the weights", flush=True)
    orc = OracleModel(eng27)
    eng27.reset(pos, tok)
    got_tok = int(eng27.generate(1)[0])
    got = eng27.logits(1)[0]
    print("27B: the oracle's 64-layer step", flush=True)
    am, want = orc.step(tok, pos)
    err = np.abs(got.astype(np.float64) - want)
    print(f"27B step: max err / max logit {err.max() / np.abs(want).max():.3e}, argmax {got_tok} vs {am}",
          flush=True)
    assert close(got, want, abs_frac=5e-4, rel_big=2e-3)
    assert argmax_ok(got_tok, want)
    c = eng27.ctrl()
    assert c[mi.CTRL_POS] == pos + 1 and c[mi.CTRL_DEBUG] == 0


@pytest.mark.parametrize("k", [3, 7])
def test_cfg2_27b_verify_rows_bitwise_plain_steps(eng27, k):
    P, t0 = 4000, 17
    eng27.reset(P, t0)
    toks, lg = [], []
    for _ in range(k + 1):
        toks.append(int(eng27.generate(1)[0]))
        lg.append(eng27.logits(1)[0].copy())
    eng27.reset(P, t0)
    print(f"27B verify k={k}", flush=True)
    rows = eng27.verify(toks[:k])
    assert list(rows) == toks
    got = eng27.logits(k + 1)
    for m in range(k + 1):
        assert np.array_equal(got[m].view(np.uint32), lg[m].view(np.uint32)), m
    # a draft list with one wrong token: accept stops there and takes that row's argmax
    # (the synthetic 27B model's fp16 residual overflows on some inputs, which the step flags and
    # verify refuses: the wrong token is the first of toks[1] + 1, + 2, ... whose rows stay finite)
    bad = list(toks[:k])
    for d in range(1, 9):
        bad[1] = (toks[1] + d) % 151936
        eng27.reset(P, t0)
        try:
            rows = eng27.verify(bad)
            break
        except mi.MiError as e:
            assert "not finite" in str(e)
            print(f"wrong token {bad[1]}: a row left the fp16 range, next", flush=True)
    else:
        pytest.fail("no finite wrong-token list in 8 tries")
    j, nxt = mi.accept_greedy(rows, bad)
    assert (j, nxt) == (1, toks[1]) and O.accept_greedy(rows, bad) == (j, nxt)
    eng27.commit(P, j, nxt)
    c = eng27.ctrl()
    assert c[mi.CTRL_POS] == P + 2 and c[mi.CTRL_CUR] == toks[1]


def _weights(K, N, seed):
    rng = np.random.default_rng(seed)
    qw = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    sc = O.f32_to_f16_bits(rng.uniform(0.002, 0.02, size=(K // 64, N)).astype(np.float32))
    return qw, sc


@pytest.mark.parametrize("name,K,N", [("gate_up", 5120, 34816), ("down", 17408, 5120), ("qkv", 5120, 7168)])
def test_cfg5_small_m_27b_shapes(name, K, N):
    qw, sc = _weights(K, N, K ^ N)
    S = mi.lib().mi_gemv_pick_s(K, N)
    dq, ds = dev(qw), dev(sc)
    x16 = O.f32_to_f16_bits(np.random.default_rng(N).standard_normal((16, K)).astype(np.float32))
    xf = O.f16_bits_to_f32(x16)
    part = empty((S, 16, N), np.float32)
    rows1 = {}
    for M in (1, 4, 8, 16):
        print(f"cfg5 {name} K={K} N={N} M={M} S={S}", flush=True)
        dx = dev(np.ascontiguousarray(x16[:M]))
        mi.call("mi_gemv_w4a16", ptr(dq), ptr(ds), ptr(dx), ptr(part), M, K, N, S, stream())
        sync()
        p = host(part, np.float32).reshape(-1)[:S * M * N].reshape(S, M, N).copy()
        got = np.zeros((M, N), np.float32)
        for s in range(S):
            got = got + p[s]
        if M == 1:
            rows1[0] = p[:, 0].copy()
        else:
            # property R: row 0 is bitwise the 1-row launch's
            assert np.array_equal(p[:, 0].view(np.uint32), rows1[0].view(np.uint32))
            ref, bound = O.gemv_ref(qw, sc, K, N, xf[:M])
            over, mr = O.n2_over(got, ref, bound)
            assert over == 0, f"N2 violated: max ratio {mr}"
            twin = O.gemv_twin(qw, sc, K, N, xf[:M], S=S).astype(np.float64)
            assert np.all(np.abs(got - twin) <= 2e-3 * np.abs(twin) + 2e-3 * np.abs(twin).max())


def test_cfg3_131072_int8_paged():
    QH, KVH, HD, Lm, P, tgt = 40, 8, 128, 131072, 64, 128
    sh = O.attn_shape(QH, KVH, HD)
    rng = np.random.default_rng(131)
    k = rng.integers(-127, 128, size=(KVH, Lm, HD)).astype(np.int8)
    v = rng.integers(-127, 128, size=(KVH, Lm, HD)).astype(np.int8)
    ks = O.f32_to_f16_bits(rng.uniform(0.005, 0.05, (KVH, Lm)).astype(np.float32))
    vs = O.f32_to_f16_bits(rng.uniform(0.005, 0.05, (KVH, Lm)).astype(np.float32))
    q = rng.standard_normal((1, QH, HD)).astype(np.float32)
    pos = Lm - 1
    a, pa = gpu_attention(sh, q, 1, k, v, ks, vs, pos, 1, tgt)
    pages = rng.permutation(Lm // P).astype(np.uint32)
    phys = (pages[:, None] * P + np.arange(P)[None, :]).ravel()
    kp, vp_ = np.empty_like(k), np.empty_like(v)
    kp[:, phys], vp_[:, phys] = k, v
    ksp, vsp = np.empty_like(ks), np.empty_like(vs)
    ksp[:, phys], vsp[:, phys] = ks, vs
    del k, v
    b, pb = gpu_attention(sh, q, 1, kp, vp_, ksp, vsp, pos, 1, tgt, pages, P)
    assert np.array_equal(a, b)
    assert np.array_equal(pa.view(np.uint32), pb.view(np.uint32))
    # fp64 softmax attention for one q head per kv head (the paged cache through the table)
    G = QH // KVH
    heads = [kv * G + (kv % G) for kv in range(KVH)]
    want = np.zeros((len(heads), HD))
    for i, h in enumerate(heads):
        O.lib().orc_attend64(C.byref(sh), O._p(np.ascontiguousarray(q[0, h])), h // G, pos + 1, 1, O.ORC_F16,
                             O._p(kp), O._p(vp_), O._p(ksp), O._p(vsp), HD, Lm * HD, 1, Lm, O._p(pages), P,
                             O._p(want[i]))
    got = a[0].reshape(QH, HD)
    check_close(got[heads], want)


def test_cfg4_full_moe_step_vs_oracle():
    """BASELINE configs[3] at full size: the captured 40-layer MoE step (router GEMV, gate||up
    with the routing in its prologue, down with the next norm, attention 16 / 2 heads of 256)
    against the oracle's MoE step (moe_ref.h:144-152, 190-304) on the same weights and cache."""
    print("cfg4: building the 40-layer MoE engine", flush=True)
    eng = mi.Engine(mi.desc_moe_cfg4(max_len=4160), seed=1235)
    eng.capture(1)
    pos, tok = 4096, 1000
    print("cfg4: oracle copies of the weights", flush=True)
    orc = OracleModel(eng)
    eng.reset(pos, tok)
    got_tok = int(eng.generate(1)[0])
    got = eng.logits(1)[0]
    print("cfg4: the oracle's 40-layer step", flush=True)
    am, want = orc.step(tok, pos)
    print(f"cfg4 step: argmax {got_tok} vs {am}", flush=True)
    assert close(got, want, abs_frac=5e-4, rel_big=2e-3)
    assert argmax_ok(got_tok, want)
    c = eng.ctrl()
    assert c[mi.CTRL_POS] == pos + 1 and c[mi.CTRL_DEBUG] == 0
    del orc
    eng.close()


def test_cfg2_27b_bf16_step_vs_oracle():
    """The 27B shape with bf16 activations (the reference's type) at seed 42, where the f16
    activations of the same synthetic model leave the f16 range in the first step: the bf16 step
    stays finite and matches the oracle's bf16 step."""
    pos, tok = 4096, 1000
    e16 = mi.Engine(mi.desc_27b(max_len=4160), seed=42)
    e16.capture(1)
    e16.reset(pos, tok)
    with pytest.raises(mi.MiError, match="not finite"):
        e16.generate(1)
    print("27B seed 42, f16 activations: the step left the f16 range (flagged)", flush=True)
    e16.close()
    print("building the bf16 27B engine", flush=True)
    eng = mi.Engine(mi.desc_27b(max_len=4160, act_bf16=1), seed=42)
    eng.capture(1)
    orc = OracleModel(eng)
    eng.reset(pos, tok)
    got_tok = int(eng.generate(1)[0])
    got = eng.logits(1)[0]
    print("27B bf16: the oracle's 64-layer step", flush=True)
    am, want = orc.step(tok, pos)
    assert np.all(np.isfinite(want)) and np.all(np.isfinite(got))
    assert close(got, want, abs_frac=5e-4, rel_big=2e-3)
    assert argmax_ok(got_tok, want)
    assert eng.ctrl()[mi.CTRL_DEBUG] == 0
    del orc
    eng.close()
