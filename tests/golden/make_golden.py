"""Writes the golden fixtures of the layer/model composition (this container only).

The upstream PyTorch YuE2 model (vendor/yue/src/yue2/modeling_yue2.py, read
from the reference checkout) is the only runnable statement of the whole
decoder layer; the closed-form and brute-force checks pin each op on its own,
but not their wiring (q/k-norm before RoPE, GQA head map, residual order).
This script loads this build's deterministic weights into that model, runs it
on CPU in bf16 and fp32, and stores only inputs' seeds and outputs:

  tiny_model.npz   2-layer model (H 256, F 512, 4/2 heads, D 128, V 512):
                   logits after a 7-token prefill and 3 teacher-forced steps
  layer_3072.npz   one 3B-shaped layer (H 3072, 24/8 heads, F 8192,
                   eps 1e-5, theta 5e5), KV cache N(0,1) for 511 slots, input
                   hidden N(0,1), decode at slot 511: output hidden

Run: python tests/golden/make_golden.py   (needs /root/reference)
"""
import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "yue2-mlx_amd"))
import yuear  # noqa: E402

REF = "/root/reference/vendor/yue/src/yue2/modeling_yue2.py"


def load_upstream():
    spec = importlib.util.spec_from_file_location("modeling_yue2", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def to_torch(arr, dtype):
    t = torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16)
    return t.to(dtype)


def bits(t):
    return t.detach().to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


TINY = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=128, vocab_size=512, max_position_embeddings=64,
            rms_norm_eps=1e-5, rope_theta=500000.0, qk_norm=True)
TINY_SEED, TINY_STD, TINY_NORM_STD = 11, 0.02, 0.1
TINY_PREFIX = [3, 17, 255, 1, 98, 400, 7]
TINY_STEPS = [12, 499, 64]

LAYER = dict(hidden_size=3072, intermediate_size=8192, num_hidden_layers=1,
             num_attention_heads=24, num_key_value_heads=8, head_dim=128, vocab_size=128,
             max_position_embeddings=1024, rms_norm_eps=1e-5, rope_theta=500000.0, qk_norm=True)
LAYER_SEED, LAYER_LEN = 1, 512
KV_STREAM, X_STREAM = 900, 901  # generator stream ids of the random cache / input


def tiny_golden(mod):
    w = yuear.random_weights(TINY, TINY_SEED, TINY_STD, TINY_NORM_STD)
    out = {}
    for dtype, tag in ((torch.bfloat16, "bf16"), (torch.float32, "f32")):
        cfg = mod.YuE2Config(**{k: v for k, v in TINY.items() if k != "qk_norm"},
                             max_latent_frames=64)
        torch.manual_seed(0)
        model = mod.YuE2ForCausalLM(cfg).eval().to(dtype)
        state = model.state_dict()
        with torch.no_grad():
            for name, arr in w.items():
                state[name].copy_(to_torch(arr, dtype).reshape(state[name].shape))
        c = TINY
        cache = mod.StaticKVCache(c["num_hidden_layers"], 1, c["num_key_value_heads"], 16,
                                  c["head_dim"], dtype, torch.device("cpu"))
        logits = []
        with torch.inference_mode():
            r = model(torch.tensor([TINY_PREFIX]), past_key_values=cache, use_cache=True,
                      logits_to_keep=1)
            logits.append(r.logits[0, -1])
            for t in TINY_STEPS:
                r = model(torch.tensor([[t]]), past_key_values=cache, use_cache=True,
                          logits_to_keep=1)
                logits.append(r.logits[0, -1])
        stack = torch.stack(logits)
        out[f"logits_{tag}"] = bits(stack) if tag == "bf16" else stack.float().numpy()
    checksum = np.uint64(0)
    for name in sorted(w):
        checksum += np.uint64(int(w[name].astype(np.uint64).sum()))
    np.savez(os.path.join(HERE, "tiny_model.npz"), prefix=np.array(TINY_PREFIX, np.int32),
             steps=np.array(TINY_STEPS, np.int32), seed=TINY_SEED, std=TINY_STD,
             norm_std=TINY_NORM_STD, weight_checksum=checksum, **out)


def layer_golden(mod):
    c = LAYER
    H, D, Hkv = c["hidden_size"], c["head_dim"], c["num_key_value_heads"]
    w = {k: v for k, v in yuear.random_weights(c, LAYER_SEED).items() if ".layers.0." in k}
    kv = yuear.random_normal(LAYER_SEED, KV_STREAM, (2, Hkv, LAYER_LEN - 1, D))
    x = yuear.random_normal(LAYER_SEED, X_STREAM, (H,))
    out = {}
    for dtype, tag in ((torch.bfloat16, "bf16"), (torch.float32, "f32")):
        cfg = mod.YuE2Config(**{k: v for k, v in c.items() if k != "qk_norm"},
                             max_latent_frames=64)
        layer = mod.DecoderLayer(cfg).eval().to(dtype)
        state = layer.state_dict()
        with torch.no_grad():
            for name, arr in w.items():
                key = name.replace("model.layers.0.", "")
                state[key].copy_(to_torch(arr, dtype).reshape(state[key].shape))
        rot = mod.RotaryEmbedding(D, c["rope_theta"])
        pos = torch.tensor([[LAYER_LEN - 1]])
        cos, sin = rot(pos)
        cache = mod.StaticKVCache(1, 1, Hkv, LAYER_LEN, D, dtype, torch.device("cpu"))
        cache.key_cache[0][0, :, :LAYER_LEN - 1] = to_torch(kv[0], dtype)
        cache.value_cache[0][0, :, :LAYER_LEN - 1] = to_torch(kv[1], dtype)
        cache._seen_tokens = LAYER_LEN - 1
        with torch.inference_mode():
            y = layer(to_torch(x, dtype).reshape(1, 1, H), cos, sin, past_key_value=cache,
                      layer_idx=0, cache_position=pos[0])
        out[f"hidden_{tag}"] = bits(y[0, 0]) if tag == "bf16" else y[0, 0].float().numpy()
    np.savez(os.path.join(HERE, "layer_3072.npz"), seed=LAYER_SEED, length=LAYER_LEN,
             kv_stream=KV_STREAM, x_stream=X_STREAM, **out)


if __name__ == "__main__":
    torch.set_num_threads(8)
    mod = load_upstream()
    tiny_golden(mod)
    layer_golden(mod)
    print("wrote", os.listdir(HERE))
