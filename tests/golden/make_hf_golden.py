"""Write golden vectors for the oracle from transformers' own LFM2 model.

    python tests/golden/make_hf_golden.py

Runs here (CPU) only; the fixtures it writes are committed data. It builds a
3-layer LFM2 (conv, conv, attention; hidden 1024, FFN 2560, 16/8 heads, head
dim 64, RoPE theta 1e6, eps 1e-5, eager attention, BF16) with a 512-row tied
vocabulary, loads the seeded synthetic weights of the package's generator
(seed 7), and decodes 8 positions token by token with the KV/conv cache, the
way experiments/010_cpu_greedy.py:46-63 drives the model. For every position
it stores, as BF16 bit patterns, the output of each decoder layer, the
logits and the argmax, plus the conv states and KV cache after the run.

Three variants are recorded:
  hf_stock   transformers as installed (its causal_conv1d_update rounds the
             3-tap conv once, through F.conv1d);
  hf_pinned  the same model with the conv step rounded per product, as the
             reference's pinned transformers 5.5.4 and its own restatement
             (experiments/006_lfm25_cpu_two_recurrent_layers.py:41-47) do;
  hf_sdpa    hf_pinned with the SDPA attention implementation, the default
             of the model class the reference's CPU path loads
             (experiments/010_cpu_greedy.py:42-44; Lfm2PreTrainedModel
             supports SDPA), where the eager variants follow
             eager_attention_forward (BF16 probabilities).
"""

from __future__ import annotations

import importlib
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
lab = importlib.import_module("ryzenai-npu-lab_amd")

OUT = Path(__file__).resolve().parent / "hf_lfm2_3layer.npz"
SEED, VOCAB, LAYERS, POSITIONS = 7, 512, 3, 8
LAYER_TYPES = ["conv", "conv", "full_attention"]


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def build_model(attn: str = "eager"):
    from transformers import Lfm2Config, Lfm2ForCausalLM
    cfg = Lfm2Config(vocab_size=VOCAB, hidden_size=1024, intermediate_size=2560,
                     num_hidden_layers=LAYERS, num_attention_heads=16, num_key_value_heads=8,
                     max_position_embeddings=4096, norm_eps=1e-5, conv_L_cache=3,
                     block_auto_adjust_ff_dim=False, layer_types=LAYER_TYPES,
                     rope_parameters={"rope_type": "default", "rope_theta": 1_000_000.0},
                     tie_word_embeddings=True)
    cfg._attn_implementation = attn
    # Instantiate under a BF16 default dtype, as from_pretrained(dtype=bf16)
    # does: parameters are BF16 while the rotary inv_freq buffer, built with an
    # explicit .float(), stays FP32 (model.to(bf16) would round it to BF16).
    previous = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        model = Lfm2ForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(previous)
    inv = model.model.rotary_emb.inv_freq
    if inv.dtype != torch.float32:
        raise RuntimeError(f"rotary inv_freq is {inv.dtype}, expected float32")
    ck = lab.weights.synthetic_checkpoint(SEED, VOCAB, layers=LAYERS)
    state = {}
    for name, arr in ck.items():
        t = torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16)
        state[name] = t
    missing, unexpected = model.load_state_dict(state, strict=False)
    missing = [m for m in missing if m != "lm_head.weight"]
    if missing or unexpected:
        raise RuntimeError(f"state mismatch: missing={missing} unexpected={unexpected}")
    model.tie_weights()
    return model


def per_product_conv_update(hidden_states, conv_state, weight, bias=None, activation=None):
    """One-token conv with every tap product rounded to BF16 before an FP32
    sum (experiments/006_lfm25_cpu_two_recurrent_layers.py:44-45)."""
    state = torch.cat([conv_state[:, :, 1:], hidden_states.to(conv_state.dtype)], dim=-1)
    conv_state.copy_(state)
    out = torch.sum(state * weight.unsqueeze(0), dim=-1, keepdim=True)
    return out.to(hidden_states.dtype)


def run(model, ids):
    from transformers.cache_utils import DynamicCache  # noqa: F401
    outs = {}
    captured = []
    hooks = [layer.register_forward_hook(lambda m, i, o: captured.append(o))
             for layer in model.model.layers]
    past = None
    with torch.inference_mode():
        for p, tok in enumerate(ids):
            captured.clear()
            res = model(torch.tensor([[tok]]), past_key_values=past, use_cache=True)
            past = res.past_key_values
            for li, o in enumerate(captured):
                h = o[0] if isinstance(o, tuple) else o
                outs[f"p{p}_layer{li}"] = bits(h.reshape(-1))
            logits = res.logits[0, -1]
            outs[f"p{p}_logits"] = bits(logits)
            outs[f"p{p}_argmax"] = np.array([int(torch.argmax(logits.float()))], dtype=np.int32)
    for h in hooks:
        h.remove()
    conv_layers = [i for i, t in enumerate(LAYER_TYPES) if t == "conv"]
    for ci, li in enumerate(conv_layers):
        outs[f"conv{ci}_state"] = bits(past.layers[li].conv_states[0].reshape(1024, -1)) \
            if hasattr(past.layers[li], "conv_states") else np.zeros(0, np.uint16)
    att = [i for i, t in enumerate(LAYER_TYPES) if t == "full_attention"]
    for ai, li in enumerate(att):
        outs[f"attn{ai}_keys"] = bits(past.layers[li].keys[0])
        outs[f"attn{ai}_values"] = bits(past.layers[li].values[0])
    return outs


def main():
    torch.manual_seed(0)
    from transformers.models.lfm2 import modeling_lfm2 as ml
    ids = [int(v) for v in lab.rng.uniform_ints(SEED, "golden.ids", POSITIONS, 9)]
    model = build_model()
    stock = run(model, ids)
    original = ml.causal_conv1d_update
    try:
        ml.causal_conv1d_update = per_product_conv_update
        for layer in model.model.layers:
            if hasattr(layer, "conv") and hasattr(layer.conv, "causal_conv1d_update"):
                layer.conv.causal_conv1d_update = per_product_conv_update
        pinned = run(build_model(), ids)
        sdpa = run(build_model("sdpa"), ids)
    finally:
        ml.causal_conv1d_update = original
    arrays = {"ids": np.array(ids, dtype=np.int32),
              "meta": np.array([SEED, VOCAB, LAYERS, POSITIONS], dtype=np.int64)}
    arrays.update({f"hf_stock.{k}": v for k, v in stock.items()})
    arrays.update({f"hf_pinned.{k}": v for k, v in pinned.items()})
    arrays.update({f"hf_sdpa.{k}": v for k, v in sdpa.items()})
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes), ids={ids}")


if __name__ == "__main__":
    main()
