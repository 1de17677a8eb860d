"""Write golden vectors by running the reference's own PyTorch modules.

Run in the container that mounts the reference (read-only, never shipped):

    python tests/golden/make_golden.py /root/reference/src

It imports ``reference/model.py``, ``reference/layers.py`` and
``reference/cache.py`` from that tree and runs them on CPU on the inputs of
tests/golden/inputs.py, for exactly the values nothing else pins: the pooled
key / block score values that feed ``topk`` (hence the selected sets), the
whole-layer plumbing with its dtype casts, and ``chunk_gated_delta_rule``'s
float32 values. Per configuration it stores, in ``tests/golden/*.npz``:

* sha256 digests of every output (the oracle must reproduce them bit for bit
  on this torch build), and strided samples of them for tolerance checks;
* the exact indexer projections and the reference's block scores and selected
  block sets, so the HIP path can be fed the same bits and must select the
  same blocks;
* the torch version and the input seeds.

The reference's ``F.linear`` and ``Tensor.topk`` are observed (wrapped for the
duration of a call, then restored) to capture projection outputs, the score
tensor handed to ``topk``, and the input of the output projection. Nothing of
the reference's source is copied into the fixtures: they are data.
"""

from __future__ import annotations

import json
import os
import sys
from contextlib import contextmanager

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import inputs as gi  # noqa: E402


class _Cfg:
    """The config fields the three token-mixing methods read."""

    hidden_size = gi.HIDDEN
    rms_norm_eps = 1e-6
    num_attention_heads = gi.QSA_HEADS
    num_kv_heads = gi.QSA_KV
    head_dim = gi.QSA_HD
    indexer_heads = gi.IDX_HEADS
    indexer_head_dim = gi.IDX_DIM
    indexer_budget = gi.BUDGET
    indexer_compress_ratio = gi.RATIO
    linear_num_v_heads = gi.DN_HV
    linear_num_k_heads = gi.DN_HK
    linear_head_dim = gi.DN_D
    conv_kernel = gi.DN_K
    linear_key_dim = gi.DN_HK * gi.DN_D
    linear_value_dim = gi.DN_HV * gi.DN_D
    conv_dim = gi.CONV_DIM
    output_gate_type = "sigmoid"


def _sample(t: torch.Tensor, n: int = 4096) -> np.ndarray:
    flat = t.detach().float().reshape(-1)
    stride = max(1, flat.numel() // n)
    return flat[::stride][:n].numpy().astype(np.float32)


@contextmanager
def _observe(store):
    """Record (weight name -> (input, output)) of F.linear and the last topk call."""
    names = {id(v): k.split(".", 2)[2] for k, v in store.weights.items()}
    seen = {"linear": {}, "topk": []}
    orig_linear, orig_topk = F.linear, torch.Tensor.topk

    def linear(x, weight, bias=None):
        y = orig_linear(x, weight, bias)
        key = names.get(id(weight))
        if key is not None:
            seen["linear"][key] = (x.detach().clone(), y.detach().clone())
        return y

    def topk(self, *a, **kw):
        res = orig_topk(self, *a, **kw)
        seen["topk"].append((self.detach().clone(), res.indices.clone()))
        return res

    F.linear = linear
    torch.Tensor.topk = topk
    try:
        yield seen
    finally:
        F.linear = orig_linear
        torch.Tensor.topk = orig_topk


def _selected_from_mask(mask: torch.Tensor, qpos0: int) -> list:
    """Per query, the eligible blocks whose tokens the mask shows."""
    out = []
    m = mask[0, 0]
    for i in range(m.shape[0]):
        p = qpos0 + i
        n_el = (p + 1) // gi.RATIO
        out.append([j for j in range(n_el) if bool(m[i, j * gi.RATIO])])
    return out


def main(ref_src: str) -> None:
    sys.path.insert(0, ref_src)
    from ttrunner_qwen38_flash_next.reference.cache import HybridCache
    from ttrunner_qwen38_flash_next.reference.layers import (
        RotaryEmbedding,
        chunk_gated_delta_rule,
        recurrent_gated_delta_rule,
    )
    from ttrunner_qwen38_flash_next.reference.model import Qwen4ExpModel

    torch.set_num_threads(8)
    rot = RotaryEmbedding(64, 1e7, [11, 11, 10])
    meta = {"torch": torch.__version__, "cpu_capability": torch.backends.cpu.get_cpu_capability()}

    def model(store):
        m = Qwen4ExpModel.__new__(Qwen4ExpModel)
        m.config = _Cfg()
        m.store = store
        m.rotary = rot
        m.probe = None
        return m

    def tables(total: int):
        pos = torch.arange(total)[None]
        return rot(pos[None].expand(3, -1, -1))

    out = {}

    # rope table digests: the oracle's RotaryEmbedding must reproduce them
    cos, sin = tables(32768)
    out["rope"] = {"cos_sha": gi.digest(cos), "sin_sha": gi.digest(sin)}

    # ---------------- config 1: fp32 plumbing, decode at 192 of 256 -------------
    def decode_layers(tag, dtype, pos, dn_seeds, qsa_seeds, hid_seed):
        res = {}
        hidden = gi.hidden_states(hid_seed, 1, dtype)
        # DeltaNet, layer 0
        wd = gi.dn_weights(0, dn_seeds[0], dtype)
        store = gi.FakeStore(wd)
        m = model(store)
        cache = HybridCache(4)
        conv, state = gi.dn_past(dn_seeds[1], dtype)
        cache[0].conv_state, cache[0].recurrent_state = conv.clone(), state.clone()
        with _observe(store) as seen:
            y = m._linear_attention(hidden, 0, cache)
        core = seen["linear"]["ssm_out.weight"][0]
        res["dn_out_sha"], res["dn_out"] = gi.digest(y), _sample(y)
        res["dn_core_sha"], res["dn_core"] = gi.digest(core), _sample(core)
        res["dn_state_sha"], res["dn_state"] = gi.digest(cache[0].recurrent_state), _sample(cache[0].recurrent_state, 65536)
        res["dn_conv_sha"] = gi.digest(cache[0].conv_state)
        # QSA, layer 3
        wq = gi.qsa_weights(3, qsa_seeds[0], dtype)
        store = gi.FakeStore(wq)
        m = model(store)
        cache = HybridCache(4)
        keys, values, idx_keys = gi.qsa_past(qsa_seeds[1], pos, dtype)
        cache[3].keys, cache[3].values, cache[3].indexer_keys = keys, values, idx_keys
        cos, sin = tables(pos + 1)
        with _observe(store) as seen:
            y = m._full_attention(hidden, 3, cos, sin, cache, pos)
        core = seen["linear"]["attn_output.weight"][0]
        res["qsa_out_sha"], res["qsa_out"] = gi.digest(y), _sample(y)
        res["qsa_core_sha"], res["qsa_core"] = gi.digest(core), core.float().reshape(-1).numpy()
        res["qsa_newk_sha"] = gi.digest(cache[3].keys[:, :, -1:])
        res["idx_q_raw"] = gi.bf16_bits(seen["linear"]["indexer.q_proj.weight"][1]) if dtype == torch.bfloat16 else seen["linear"]["indexer.q_proj.weight"][1].numpy()
        res["idx_k_raw"] = gi.bf16_bits(seen["linear"]["indexer.k_proj.weight"][1]) if dtype == torch.bfloat16 else seen["linear"]["indexer.k_proj.weight"][1].numpy()
        if seen["topk"]:
            sc, ch = seen["topk"][-1]
            res["scores"] = sc.reshape(-1).numpy().astype(np.float32)
            res["topk_torch"] = ch.reshape(-1).numpy().astype(np.int64)
        mask = None
        # the mask itself, recomputed through the reference for the selected set
        cache2 = HybridCache(4)
        cache2[3].indexer_keys = idx_keys
        mask = m._indexer_mask(hidden, 3, cos, sin, cache2, pos + 1, pos)
        res["selected"] = np.array(_selected_from_mask(mask, pos)[0], np.int64)
        meta[tag] = {"dtype": str(dtype), "pos": pos, "dn_seeds": dn_seeds, "qsa_seeds": qsa_seeds, "hidden_seed": hid_seed}
        return res

    out["cfg1"] = decode_layers("cfg1", torch.float32, 192, (100, 200), (101, 201), 11)
    out["cfg3"] = decode_layers("cfg3", torch.bfloat16, 8128, (113, 213), (103, 303), 13)
    out["cfg3b"] = decode_layers("cfg3b", torch.bfloat16, 4032, (114, 214), (104, 304), 14)

    # ---------------- config 4: delta rule, 4096 tokens -----------------------
    q, k, v, g, beta = gi.delta_rule_inputs(404, 4096)
    s0 = gi.dn_past(405)[1]
    o_c, s_c = chunk_gated_delta_rule(q, k, v, g, beta, initial_state=s0)
    o_r, s_r = recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=s0)
    out["cfg4"] = {
        "chunk_out_sha": gi.digest(o_c), "chunk_out": _sample(o_c, 65536),
        "chunk_state_sha": gi.digest(s_c), "chunk_state": _sample(s_c, 65536),
        "rec_out_sha": gi.digest(o_r), "rec_out": _sample(o_r, 65536),
        "rec_state_sha": gi.digest(s_r), "rec_state": _sample(s_r, 65536),
    }
    meta["cfg4"] = {"seed": 404, "state_seed": 405, "seq": 4096}

    # ---------------- config 5: 128-token prefill chunk at 32640 --------------
    past, seq = 32640, 128
    dtype = torch.bfloat16
    hidden = gi.hidden_states(15, seq, dtype)
    wq = gi.qsa_weights(3, 105, dtype)
    store = gi.FakeStore(wq)
    m = model(store)
    cache = HybridCache(4)
    keys, values, idx_keys = gi.qsa_past(505, past, dtype)
    cache[3].keys, cache[3].values, cache[3].indexer_keys = keys, values, idx_keys
    cos, sin = tables(past + seq)
    with _observe(store) as seen:
        y = m._full_attention(hidden, 3, cos, sin, cache, past)
    core = seen["linear"]["attn_output.weight"][0]
    sc, ch = seen["topk"][-1]
    cache2 = HybridCache(4)
    cache2[3].indexer_keys = idx_keys
    mask = m._indexer_mask(hidden, 3, cos, sin, cache2, past + seq, past)
    sel = _selected_from_mask(mask, past)
    res = {
        "qsa_out_sha": gi.digest(y), "qsa_out": _sample(y, 65536),
        "qsa_core_sha": gi.digest(core), "qsa_core": _sample(core, 65536),
        "idx_q_raw": gi.bf16_bits(seen["linear"]["indexer.q_proj.weight"][1]),
        "idx_k_raw": gi.bf16_bits(seen["linear"]["indexer.k_proj.weight"][1]),
        "scores": sc.reshape(seq, -1).numpy().astype(np.float32),
        "selected": np.array([s + [-1] * (32 - len(s)) for s in sel], np.int64),
    }
    wd = gi.dn_weights(0, 106, dtype)
    store = gi.FakeStore(wd)
    m = model(store)
    cache = HybridCache(4)
    conv, state = gi.dn_past(506, dtype)
    cache[0].conv_state, cache[0].recurrent_state = conv.clone(), state.clone()
    with _observe(store) as seen:
        y = m._linear_attention(hidden, 0, cache)
    core = seen["linear"]["ssm_out.weight"][0]
    res.update({
        "dn_out_sha": gi.digest(y), "dn_out": _sample(y, 65536),
        "dn_core_sha": gi.digest(core), "dn_core": _sample(core, 65536),
        "dn_state_sha": gi.digest(cache[0].recurrent_state), "dn_state": _sample(cache[0].recurrent_state, 65536),
        "dn_conv_sha": gi.digest(cache[0].conv_state),
    })
    out["cfg5"] = res
    meta["cfg5"] = {"past": past, "seq": seq, "qsa_seeds": (105, 505), "dn_seeds": (106, 506), "hidden_seed": 15}

    for name, arrays in out.items():
        strs = {k: v for k, v in arrays.items() if isinstance(v, str)}
        nums = {k: v for k, v in arrays.items() if not isinstance(v, str)}
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **nums)
        meta.setdefault("digests", {})[name] = strs
    with open(os.path.join(HERE, "golden_meta.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print("wrote", sorted(out))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
