"""The C-ABI library loads and exports every function include/mi355x_decode.h declares.
No compute calls (this runs without a GPU)."""
import ctypes as C
import os

import pytest

from mipkg import mi


def test_library_exports_every_declared_function():
    L = mi.lib()
    names = mi.header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_signatures_cover_the_header():
    names = set(mi.header_functions())
    assert names == set(mi.SIGNATURES), (names ^ set(mi.SIGNATURES))


def test_argument_errors_are_reported_without_a_gpu():
    L = mi.lib()
    rc = L.mi_gemv_w4a16(None, None, None, None, 1, 64, 64, 1, None)
    assert rc == -1
    assert b"null" in L.mi_last_error()
    rc = L.mi_gemv_w4a16(8, 8, 8, 8, 1, 100, 64, 1, None)
    assert rc == -2
    assert L.mi_gemv_pick_s(5120, 5120) >= 1


def test_split_k_choices_for_the_27b_shapes():
    """Measured best S on MI355X at M = 1 (qkv, o, gate_up, down, lm_head), plain and fused
    alike except RESID (at least 5 k-groups per split: o 16); S always divides K/64."""
    L = mi.lib()
    shapes = [(5120, 7168, 20), (5120, 5120, 20), (5120, 34816, 10), (17408, 5120, 34), (5120, 151936, 10)]
    for K, N, want in shapes:
        assert L.mi_gemv_pick_s(K, N) == want
        assert L.mi_gemv_pick_s_ex(K, N, mi.EPI_PARTIALS) == want
        for epi in (mi.EPI_SILU, mi.EPI_LOGITS, mi.EPI_F16OUT):
            assert L.mi_gemv_pick_s_ex(K, N, epi) == want
    assert L.mi_gemv_pick_s_ex(5120, 5120, mi.EPI_RESID) == 16  # the 27B o
    assert L.mi_gemv_pick_s_ex(17408, 5120, mi.EPI_RESID) == 34  # the 27B down
    assert L.mi_gemv_pick_s_ex(5120, 7168, mi.EPI_QKV) == 10  # the 27B qkv, fused with attn_prep
    assert L.mi_gemv_pick_s_ex(2048, 4608, mi.EPI_QKV) == 4
    for K in (64, 128, 512, 1024, 3072, 8192, 17408):
        for N in (64, 512, 4096):
            for epi in range(4):
                s = L.mi_gemv_pick_s_ex(K, N, epi)
                assert 1 <= s <= K // 64 and (K // 64) % s == 0


def test_moe_argument_errors_without_a_gpu():
    L = mi.lib()
    assert L.mi_moe_route(None, None, 1, 256, 8, 272, None) == -1
    assert L.mi_moe_route(8, 8, 1, 100, 8, 272, None) == -2      # experts not a power of two
    assert L.mi_moe_route(8, 8, 1, 256, 9, 272, None) == -2      # top_k > 8
    assert L.mi_moe_route(8, 8, 1, 256, 8, 256, None) == -2      # router_n < experts + 1
    assert L.mi_moe_gate_up(8, 8, 8, 8, 1, 256, 8, 2000, 512, None) == -2  # hidden % 512
    assert L.mi_moe_gate_up_routed(None, 272, 8, 8, 8, 8, 1, 256, 8, 2048, 512, None) == -1
    assert L.mi_moe_down_norm(8, 8, 8, 8, 1, 256, 8, 2048, 512, 8, 8, None, 1e-6, None, None, 0, 0, None) == -1
    assert L.mi_moe_down_norm(16, 16, 16, 16, 9, 256, 8, 2048, 512, 16, 16, None, 1e-6, 16, None, 0, 0, None) == -2
    assert L.mi_moe_gate_up_routed(8, 256, 8, 8, 8, 8, 1, 256, 8, 2048, 512, None) == -2  # router_n < E + 1
    assert L.mi_moe_gate_up_routed(8, 272, 8, 8, 8, 8, 1, 256, 8, 2000, 512, None) == -2  # hidden % 512
    assert L.mi_moe_down(8, 8, 8, 8, 1, 256, 8, 2048, 2048, None) == -2    # inter > 1024
    assert L.mi_gemv_f16w(8, 16, 8, 1, 2048, 272, 3, None) == -2           # ksplit not 2^n
    assert b"ksplit" in L.mi_last_error()
    assert L.mi_moe_route(8, 8, 65536, 256, 8, 272, None) == -2    # more rows than the grid takes
    assert L.mi_gemv_f16w(16, 16, 8, 65536, 2048, 272, 16, None) == -2
    # the grouped expert FFN of a prefill chunk: T 1..2048, the decode kernels' shape limits
    a = [16] * 5
    w = [16, 16, 16, 16, 16, None]
    assert L.mi_moe_prefill(None, *a[1:], 4, 256, 8, 2048, 512, *w) == -1
    assert L.mi_moe_prefill(*a, 2049, 256, 8, 2048, 512, *w) == -2
    assert L.mi_moe_prefill(*a, 4, 100, 8, 2048, 512, *w) == -2
    assert L.mi_moe_prefill(*a, 4, 256, 9, 2048, 512, *w) == -2
    assert L.mi_moe_prefill(*a, 4, 256, 8, 2000, 512, *w) == -2
    assert L.mi_moe_prefill(*a, 4, 256, 8, 2048, 2048, *w) == -2
    assert b"moe_prefill" in L.mi_last_error()


def test_kv8_argument_errors_without_a_gpu():
    """The int8 writer and the rotated reduce are defined for head_dim 256 only
    (src/common/kv8.h kHeadDim); the checks run before any launch."""
    L = mi.lib()
    sh = mi.AttnShape(40, 8, 128, 128, 0, 7168, 5120, 6144, 0.08838835, 1e-6)
    assert L.mi_attn_reduce_kv8(8, 8, None, 8, 1, 8, 0, mi.shape_ref(sh), None) == -2
    assert b"head_dim 256" in L.mi_last_error()
    assert L.mi_attn_prep_kv8(8, 8, 1, 1, mi.shape_ref(sh), None, None, 8, 8, None, 8, 8, 8, 8, 128, 128, 1, 1,
                              None, 0, 0, None) == -2
    sh.head_dim = 256
    assert L.mi_attn_prep_kv8(8, 8, 1, 1, mi.shape_ref(sh), None, None, 8, 8, None, 8, 8, None, 8, 256, 256, 1, 1,
                              None, 0, 0, None) == -1   # no k_scale


def test_engine_rejects_int8_kv_off_head_dim_256():
    """The int8 rotated cache needs head_dim 256; the shape check runs before any HIP call."""
    L = mi.lib()
    d = mi.dense_desc(2, 512, 8, 2, 128, 1024, 4096, 512, kv_int8=1)
    assert not L.mi_engine_create(C.byref(d), 1, None)
    assert b"unsupported model shape" in L.mi_last_error()


def test_prefill_and_handoff_argument_errors_without_a_gpu():
    """The prefill kernels' and the hand-off initialiser's argument checks run before any launch."""
    import oracle as O
    L = mi.lib()
    assert L.mi_gemv_handoff_init(None, 16, None) == -1
    assert L.mi_gemm_w4a16(16, 16, 16, 16, 4, 96, 128, None) == -2       # K not a multiple of 64
    assert L.mi_gemm_w4a16(16, 16, 16, 16, 4, 128, 96, None) == -2       # N not a multiple of 128
    assert L.mi_gemm_w4a16_silu(None, 16, 16, 16, 4, 128, 128, None) == -1
    sh = O.attn_shape(8, 2, 64)
    assert L.mi_attn_prefill(16, 16, 16, 64, 64, None, 0, 4, 0, mi.shape_ref(sh), 16, None) == -2  # head_dim 64
    sh = O.attn_shape(8, 2, 128, gated=True)
    assert L.mi_attn_prep_rows(16, 4, 0, mi.shape_ref(sh), None, None, 16, 16, 16, 16, 128, 128, None, 0, None) == -2
    sh = O.attn_shape(16, 2, 128)
    assert L.mi_attn_prefill_kv8(16, 16, 16, 16, 16, 128, 128, 1, 128, None, 0, 4, 0, mi.shape_ref(sh), 16, 16,
                                 None) == -2  # the rotation needs head_dim 256
    assert L.mi_engine_prefill(None, None, 0, 0) == -1


def test_argmax_static_rejects_sizes_beyond_its_scratch():
    """mi_argmax_static's device array holds 8192 chunk winners: ceil(vocab / 1024) * M above
    that is refused before anything touches a GPU."""
    L = mi.lib()
    assert L.mi_argmax_static(8, 8, None, 0, 8, 1025 * 1024, 1024, None) == -2
    assert b"8192" in L.mi_last_error()
    assert L.mi_argmax_static(None, 8, None, 0, 1, 1024, 1024, None) == -1



def test_verify_attention_bind_rule():
    """verify_attn.h:93-100 at 16 q / 2 kv heads: the many-row kernel at 16, 32, 64 rows of an
    f16 cache only"""
    L = mi.lib()
    assert [L.mi_attn_verify_binds(M, 0, 16, 2) for M in (1, 2, 4, 8, 15, 16, 32, 64, 65)] == \
        [0, 0, 0, 0, 0, 1, 1, 1, 0]
    assert L.mi_attn_verify_binds(16, 1, 16, 2) == 0     # int8 cache: the decode kernel
    assert L.mi_attn_verify_binds(16, 0, 40, 8) == 0     # other heads


def test_mtp_head_shape_rules_without_a_gpu():
    """engine_create refuses more than one MTP head before touching the device."""
    import ctypes as C
    L = mi.lib()
    d = mi.dense_desc(2, 512, 8, 2, 256, 1024, 4096, 512, mtp=2)
    assert not L.mi_engine_create(C.byref(d), 1, None)
    assert b"unsupported model shape" in L.mi_last_error()


def test_int8_head_quantiser_is_the_oracles():
    """mi_lm_head_int8_quantise (the product's load-time quantiser, host code) bitwise the
    oracle's row quantiser at every element of its layout, which is a bijection onto K N
    bytes."""
    import numpy as np
    import oracle as O
    L = mi.lib()
    K, N = 256, 48
    rng = np.random.default_rng(2)
    w = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
    w[4] = 0
    w[9, 3] = -2.0
    qt = np.zeros(K * N, np.int8)
    st = np.zeros(N, np.float32)
    assert L.mi_lm_head_int8_quantise(w.ctypes.data, K, N, qt.ctypes.data, st.ctypes.data) == 0
    idx = np.array([[L.mi_i8w_index(K, k, n) for k in range(K)] for n in range(N)])
    assert np.array_equal(np.sort(idx.ravel()), np.arange(K * N))
    for n in range(N):
        q = np.zeros(K, np.int8)
        s = O.lib().orc_quantise_row_int8(O._p(np.ascontiguousarray(w[n])), K, O._p(q))
        assert np.float32(s).view(np.uint32) == st[n].view(np.uint32)
        assert np.array_equal(qt[idx[n]], q)
    assert L.mi_lm_head_int8_quantise(w.ctypes.data, 100, N, qt.ctypes.data, st.ctypes.data) == -1
