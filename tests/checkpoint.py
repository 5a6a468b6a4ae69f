"""A small Qwen2-style checkpoint on disk: config.json + model.safetensors.

TEST INFRASTRUCTURE. Written with numpy alone, byte by byte from the published
safetensors layout (an 8-byte little-endian header length, a JSON header of
{name: {"dtype", "shape", "data_offsets"}}, then the tensor bytes; offsets are
relative to the end of the header), so the reader it exercises -- the
reference's own loader (src/safetensors.cpp, src/weights.cpp:89-117,
src/config.cpp) -- is checked against an independent writer.

The model has the layer shape the HIP kernels serve (hidden 896, 14 query / 2
KV heads of 64) with a small MLP and vocabulary, so the file stays a few MB:
tensor names follow the Hugging Face Qwen2 convention the reference loads
(model.embed_tokens.weight, model.layers.N.self_attn.q_proj.weight/.bias, ...,
lm_head.weight when the embeddings are untied). Matrices, norms and biases are
stored as BF16 (round to nearest even), like the published checkpoints.
"""
import json
import os
import struct

import numpy as np

HIDDEN, HEADS, KV_HEADS, HEAD_DIM = 896, 14, 2, 64


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def tensors(seed: int, layers: int, inter: int, vocab: int, tie: bool) -> dict:
    """Seeded weights of the checkpoint, as float32 arrays keyed by tensor name."""
    rng = np.random.default_rng(seed)
    q_dim, kv_dim = HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM

    def mat(rows, cols, s):
        return (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(s))

    def vec(n, base, s):
        return (np.float32(base) + rng.standard_normal(n, dtype=np.float32) * np.float32(s))

    t = {"model.embed_tokens.weight": mat(vocab, HIDDEN, 1.0),
         "model.norm.weight": vec(HIDDEN, 1.0, 0.1)}
    if not tie:
        t["lm_head.weight"] = mat(vocab, HIDDEN, 0.05)
    for l in range(layers):
        p = f"model.layers.{l}."
        t[p + "input_layernorm.weight"] = vec(HIDDEN, 1.0, 0.1)
        t[p + "post_attention_layernorm.weight"] = vec(HIDDEN, 1.0, 0.1)
        t[p + "self_attn.q_proj.weight"] = mat(q_dim, HIDDEN, 0.04)
        t[p + "self_attn.q_proj.bias"] = vec(q_dim, 0.0, 0.1)
        t[p + "self_attn.k_proj.weight"] = mat(kv_dim, HIDDEN, 0.04)
        t[p + "self_attn.k_proj.bias"] = vec(kv_dim, 0.0, 0.1)
        t[p + "self_attn.v_proj.weight"] = mat(kv_dim, HIDDEN, 0.04)
        t[p + "self_attn.v_proj.bias"] = vec(kv_dim, 0.0, 0.1)
        t[p + "self_attn.o_proj.weight"] = mat(HIDDEN, q_dim, 0.03)
        t[p + "mlp.gate_proj.weight"] = mat(inter, HIDDEN, 0.05)
        t[p + "mlp.up_proj.weight"] = mat(inter, HIDDEN, 0.05)
        t[p + "mlp.down_proj.weight"] = mat(HIDDEN, inter, 0.05)
    return t


def write_checkpoint(out_dir: str, seed: int = 11, layers: int = 2, inter: int = 512,
                     vocab: int = 768, tie: bool = False) -> dict:
    """Writes out_dir/config.json and out_dir/model.safetensors; returns the float32
    tensors (before BF16 rounding) keyed by name."""
    os.makedirs(out_dir, exist_ok=True)
    t = tensors(seed, layers, inter, vocab, tie)
    header, blobs, off = {}, [], 0
    for name in sorted(t):
        data = bf16_bits(t[name]).tobytes()
        header[name] = {"dtype": "BF16", "shape": list(t[name].shape),
                        "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    header["__metadata__"] = {"format": "pt"}
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * (-len(hj) % 8)  # the data region starts 8-byte aligned
    with open(os.path.join(out_dir, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)
    cfg = {"architectures": ["Qwen2ForCausalLM"], "model_type": "qwen2",
           "hidden_size": HIDDEN, "intermediate_size": inter, "num_hidden_layers": layers,
           "num_attention_heads": HEADS, "num_key_value_heads": KV_HEADS,
           "vocab_size": vocab, "max_position_embeddings": 32768, "rms_norm_eps": 1e-6,
           "rope_theta": 1000000.0, "tie_word_embeddings": tie, "torch_dtype": "bfloat16"}
    with open(os.path.join(out_dir, "config.json"), "w") as f:
        json.dump(cfg, f, indent=1)
    return t
