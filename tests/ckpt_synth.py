"""Synthetic GPTQ / AutoRound int4 g64 checkpoints for the loader tests: config.json plus a
safetensors file written here byte by byte (an 8-byte header length, a JSON header, the raw
little-endian tensors), so BF16 needs no framework. Shapes and names are a Qwen3-style
decoder (HF naming), dense or MoE with one shared expert (Qwen2-MoE naming)."""
import json
import os
import struct

import numpy as np

import oracle as O

_CODE = {np.dtype(np.float32): "F32", np.dtype(np.int32): "I32", np.dtype(np.uint32): "I32",
         np.dtype(np.uint8): "U8", np.dtype(np.int8): "I8"}


def write_safetensors(path, tensors):
    """tensors: name -> (dtype code, numpy array); BF16 / F16 arrays are uint16 bit patterns."""
    header, blobs, off = {}, [], 0
    for name, (code, arr) in tensors.items():
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": code, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)  # keep the data section 8-byte aligned
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def bf16(a):
    return O.f32_to_bf16_bits(np.asarray(a, np.float32))


def f16(a):
    return O.f32_to_f16_bits(np.asarray(a, np.float32))


class Synth:
    """A random checkpoint plus the float values the loader must reproduce."""

    def __init__(self, path, seed=0, layers=2, H=512, QH=8, KVH=2, HD=128, I=1024, V=4000, qk_norm=True,
                 experts=0, top_k=4, moe_inter=128, head="int4", norm_dtype="BF16", tie=False,
                 qzeros=True, g_idx=True, prefix="model.", mtp=False):
        rng = np.random.default_rng(seed)
        os.makedirs(path, exist_ok=True)
        self.path = path
        self.t = {}
        self.d = dict(layers=layers, H=H, QH=QH, KVH=KVH, HD=HD, I=I, V=V, experts=experts, top_k=top_k,
                      moe_inter=moe_inter)

        def lin(name, K, N):
            q = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
            s = f16(rng.uniform(0.004, 0.03, (K // 64, N)))
            self.t[name + ".qweight"] = ("I32", q.view(np.int32))
            self.t[name + ".scales"] = ("F16", s)
            if qzeros:
                self.t[name + ".qzeros"] = ("I32", np.full((K // 64, N // 8), 0x77777777, np.uint32).view(np.int32))
            if g_idx:
                self.t[name + ".g_idx"] = ("I32", (np.arange(K) // 64).astype(np.int32))
            return q, s

        def vec(name, n, mean=1.0, sd=0.02):
            v = (mean + sd * rng.standard_normal(n)).astype(np.float32)
            if norm_dtype == "BF16":
                b = bf16(v)
                self.t[name] = ("BF16", b)
                return O.bf16_bits_to_f32(b)
            if norm_dtype == "F16":
                b = f16(v)
                self.t[name] = ("F16", b)
                return O.f16_bits_to_f32(b)
            self.t[name] = ("F32", v)
            return v

        p = prefix
        emb = bf16(rng.standard_normal((V, H)))
        self.t[p + "embed_tokens.weight"] = ("BF16", emb)
        self.embed = O.bf16_bits_to_f32(emb)
        self.final_norm = vec(p + "norm.weight", H)
        self.layers = []
        for li in range(layers):
            lp = f"{p}layers.{li}."
            L = {}
            L["q"] = lin(lp + "self_attn.q_proj", H, QH * HD)
            L["k"] = lin(lp + "self_attn.k_proj", H, KVH * HD)
            L["v"] = lin(lp + "self_attn.v_proj", H, KVH * HD)
            L["o"] = lin(lp + "self_attn.o_proj", QH * HD, H)
            L["in_norm"] = vec(lp + "input_layernorm.weight", H)
            L["post_norm"] = vec(lp + "post_attention_layernorm.weight", H)
            if qk_norm:
                L["q_norm"] = vec(lp + "self_attn.q_norm.weight", HD)
                L["k_norm"] = vec(lp + "self_attn.k_norm.weight", HD)
            if experts:
                rw = bf16(0.05 * rng.standard_normal((experts, H)))
                sg = bf16(0.05 * rng.standard_normal((1, H)))
                self.t[lp + "mlp.gate.weight"] = ("BF16", rw)
                self.t[lp + "mlp.shared_expert_gate.weight"] = ("BF16", sg)
                L["router"] = np.concatenate([O.bf16_bits_to_f32(rw), O.bf16_bits_to_f32(sg)])
                L["experts"] = []
                for e in range(experts + 1):
                    ep = lp + (f"mlp.experts.{e}." if e < experts else "mlp.shared_expert.")
                    L["experts"].append((lin(ep + "gate_proj", H, moe_inter), lin(ep + "up_proj", H, moe_inter),
                                         lin(ep + "down_proj", moe_inter, H)))
            else:
                L["gate"] = lin(lp + "mlp.gate_proj", H, I)
                L["up"] = lin(lp + "mlp.up_proj", H, I)
                L["down"] = lin(lp + "mlp.down_proj", I, H)
            self.layers.append(L)
        if mtp:  # a dense MTP head in bf16 (the published checkpoints' form): 15 mtp.* tensors
            def wbf(name, N, K, sd=0.05):
                b = bf16(sd * rng.standard_normal((N, K)))
                self.t[name] = ("BF16", b)
                return b
            self.mtp = {"fc": wbf("mtp.fc.weight", H, 2 * H),
                        "pre_e": vec("mtp.pre_fc_norm_embedding.weight", H),
                        "pre_h": vec("mtp.pre_fc_norm_hidden.weight", H),
                        "final": vec("mtp.norm.weight", H)}
            mp = "mtp.layers.0."
            self.mtp.update({"q": wbf(mp + "self_attn.q_proj.weight", QH * HD, H),
                             "k": wbf(mp + "self_attn.k_proj.weight", KVH * HD, H),
                             "v": wbf(mp + "self_attn.v_proj.weight", KVH * HD, H),
                             "o": wbf(mp + "self_attn.o_proj.weight", H, QH * HD),
                             "in_norm": vec(mp + "input_layernorm.weight", H),
                             "post_norm": vec(mp + "post_attention_layernorm.weight", H)})
            if experts:  # an MoE model's head (spec 15e): one MoE layer, its linears in bf16
                self.mtp["router"] = np.concatenate([O.bf16_bits_to_f32(wbf(mp + "mlp.gate.weight", experts, H)),
                                                     O.bf16_bits_to_f32(wbf(mp + "mlp.shared_expert_gate.weight", 1,
                                                                            H))])
                self.mtp["experts"] = []
                for e in range(experts + 1):
                    ep = mp + (f"mlp.experts.{e}." if e < experts else "mlp.shared_expert.")
                    self.mtp["experts"].append((wbf(ep + "gate_proj.weight", moe_inter, H),
                                                wbf(ep + "up_proj.weight", moe_inter, H),
                                                wbf(ep + "down_proj.weight", H, moe_inter)))
            else:
                self.mtp.update({"gate": wbf(mp + "mlp.gate_proj.weight", I, H),
                                 "up": wbf(mp + "mlp.up_proj.weight", I, H),
                                 "down": wbf(mp + "mlp.down_proj.weight", H, I)})
            if qk_norm:
                self.mtp["q_norm"] = vec(mp + "self_attn.q_norm.weight", HD)
                self.mtp["k_norm"] = vec(mp + "self_attn.k_norm.weight", HD)
        self.head = head
        if head == "int4":
            self.lm = lin("lm_head", H, V)
        elif head == "bf16" and not tie:
            w = bf16(0.05 * rng.standard_normal((V, H)))
            self.t["lm_head.weight"] = ("BF16", w)
            self.lm_w = O.bf16_bits_to_f32(w)
        else:
            self.lm_w = self.embed
        qc = {"quant_method": "auto-round", "packing_format": "auto_round:auto_gptq", "bits": 4,
              "group_size": 64, "sym": True, "desc_act": False}
        cfg = {"architectures": ["Qwen3ForCausalLM"], "num_hidden_layers": layers, "hidden_size": H,
               "num_attention_heads": QH, "num_key_value_heads": KVH, "head_dim": HD, "intermediate_size": I,
               "vocab_size": V, "rope_theta": 1e6, "rms_norm_eps": 1e-6, "tie_word_embeddings": tie,
               "quantization_config": qc}
        if experts:
            cfg.update({"num_experts": experts, "num_experts_per_tok": top_k, "moe_intermediate_size": moe_inter,
                        "shared_expert_intermediate_size": moe_inter})
        self.cfg = cfg

    def write(self, split=1):
        names = list(self.t)
        for f in os.listdir(self.path):
            if f.endswith(".safetensors"):
                os.remove(os.path.join(self.path, f))
        per = (len(names) + split - 1) // split
        for i in range(split):
            part = {n: self.t[n] for n in names[i * per:(i + 1) * per]}
            write_safetensors(os.path.join(self.path, f"model-{i + 1:05d}-of-{split:05d}.safetensors"), part)
        with open(os.path.join(self.path, "config.json"), "w") as f:
            json.dump(self.cfg, f)
        return self.path
