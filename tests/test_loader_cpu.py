"""The checkpoint loader's host side without a GPU (src/loader/quant.cc, loader.cc;
docs/13-loader.md): config.json -> model description, and the quantisation checks
(QuantConfig::parse, assert_quant_invariants) on synthetic GPTQ / AutoRound checkpoints,
each refusal naming the offending tensor and element."""
import json
import os

import numpy as np
import pytest

from ckpt_synth import Synth
from mipkg import mi


def _err(fn):
    with pytest.raises(mi.MiError) as e:
        fn()
    return str(e.value)


def test_desc_from_config_dense_and_moe(tmp_path):
    s = Synth(str(tmp_path / "d"), V=4000, qk_norm=True).write(split=3)
    d = mi.checkpoint_desc(s, max_len=1024, max_rows=4)
    assert (d.layers, d.hidden, d.q_heads, d.kv_heads, d.head_dim, d.rot_dim) == (2, 512, 8, 2, 128, 128)
    assert (d.inter, d.vocab, d.vocab_used, d.max_len, d.max_rows) == (1024, 4032, 4000, 1024, 4)
    assert d.qk_norm == 1 and d.experts == 0 and abs(d.rope_theta - 1e6) < 1 and abs(d.rms_eps - 1e-6) < 1e-12
    m = Synth(str(tmp_path / "m"), experts=16, top_k=4, moe_inter=128, qk_norm=False, V=4096).write()
    dm = mi.checkpoint_desc(m, max_len=512)
    assert (dm.experts, dm.top_k, dm.moe_inter, dm.inter, dm.qk_norm, dm.vocab) == (16, 4, 128, 0, 0, 4096)


def test_checks_pass_and_report(tmp_path):
    s = Synth(str(tmp_path / "c")).write(split=2)
    rep = mi.checkpoint_check(s)
    # 2 layers x 7 linears + lm_head, each with qzeros and g_idx
    assert rep.startswith("15 int4 linears; 15 qzeros + 15 g_idx checked")


@pytest.mark.parametrize("field,value,msg", [
    ("bits", 8, "bits must be 4"),
    ("group_size", 128, "group_size must be 64"),
    ("sym", False, "sym must be true"),
    ("desc_act", True, "desc_act must be false"),
    ("packing_format", "auto_round:auto_awq", "not GPTQ packing"),
    ("quant_method", "awq", "quant_method"),
])
def test_quant_config_refusals(tmp_path, field, value, msg):
    syn = Synth(str(tmp_path / "q"), layers=1)
    syn.cfg["quantization_config"][field] = value
    s = syn.write()
    assert msg in _err(lambda: mi.checkpoint_check(s))


def test_data_invariant_refusals(tmp_path):
    base = "model.layers.0.self_attn.k_proj"
    # a qzeros word other than 0x77777777 (asymmetric)
    syn = Synth(str(tmp_path / "z"), layers=1)
    code, z = syn.t[base + ".qzeros"]
    z = z.copy().view(np.uint32)
    z[3, 1] = 0x77777778
    syn.t[base + ".qzeros"] = (code, z.view(np.int32))
    e = _err(lambda: mi.checkpoint_check(syn.write()))
    assert base + ".qzeros[" + str(3 * z.shape[1] + 1) + "] = 0x77777778" in e
    # a g_idx that is not the identity (activation order)
    syn = Synth(str(tmp_path / "g"), layers=1)
    code, g = syn.t[base + ".g_idx"]
    g = g.copy()
    g[70] = 0
    syn.t[base + ".g_idx"] = (code, g)
    assert base + ".g_idx[70] = 0" in _err(lambda: mi.checkpoint_check(syn.write()))
    # a non-finite scale
    syn = Synth(str(tmp_path / "n"), layers=1)
    code, sc = syn.t[base + ".scales"]
    sc = sc.copy()
    sc[1, 5] = 0x7C00
    syn.t[base + ".scales"] = (code, sc)
    assert "not a finite f16" in _err(lambda: mi.checkpoint_check(syn.write()))
    # wrong qweight shape
    syn = Synth(str(tmp_path / "w"), layers=1)
    code, q = syn.t[base + ".qweight"]
    syn.t[base + ".scales"] = ("F16", syn.t[base + ".scales"][1][:, :64])
    assert base + ".scales: expected F16" in _err(lambda: mi.checkpoint_check(syn.write()))


def test_undeclared_desc_act_needs_no_g_idx(tmp_path):
    """quant.cc: an absent desc_act is inferred false only when the checkpoint ships no g_idx."""
    syn = Synth(str(tmp_path / "a"), layers=1, g_idx=False)
    del syn.cfg["quantization_config"]["desc_act"]
    assert mi.checkpoint_check(syn.write()).endswith("subnormal scales")
    syn = Synth(str(tmp_path / "b"), layers=1, g_idx=True)
    del syn.cfg["quantization_config"]["desc_act"]
    assert "declares no desc_act" in _err(lambda: mi.checkpoint_check(syn.write()))


def test_subnormal_scales_counted_not_refused(tmp_path):
    syn = Synth(str(tmp_path / "s"), layers=1)
    base = "model.layers.0.mlp.down_proj"
    code, sc = syn.t[base + ".scales"]
    sc = sc.copy()
    sc[0, :3] = [0x00A8, 0x0001, 0x03FF]
    syn.t[base + ".scales"] = (code, sc)
    rep = mi.checkpoint_check(syn.write())
    assert rep.endswith("3 subnormal scales")


def test_bad_files_are_refused(tmp_path):
    d = tmp_path / "bad"
    d.mkdir()
    (d / "config.json").write_text("{}")
    assert "no .safetensors" in _err(lambda: mi.checkpoint_check(str(d)))
    (d / "x.safetensors").write_bytes(b"\x0a\x00\x00\x00\x00\x00\x00\x00{not json}")
    assert "bad safetensors header" in _err(lambda: mi.checkpoint_check(str(d)))
    hdr = json.dumps({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 64]}}).encode()
    (d / "x.safetensors").write_bytes(len(hdr).to_bytes(8, "little") + hdr + b"\0" * 16)
    assert "runs past the file" in _err(lambda: mi.checkpoint_check(str(d)))
