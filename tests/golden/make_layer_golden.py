"""Writes tests/golden/layer_qwen05b.npz: one decoder layer composed from the
reference's own numpy primitives.

The composition is the one of /root/reference/tools/reference_layer0.py
main() (:107-170): input RMSNorm, q/k/v projections with bias, NeoX RoPE on
q and k, causal GQA attention (kv head = h // group) with softmax, O
projection, residual, post-attention RMSNorm, silu(gate) * up, down
projection, residual. rmsnorm, softmax and silu are imported from that file
(it imports only numpy at module level); main() itself is not run (it needs a
checkpoint and a tokenizer). The projections use the INT4 weights
dequantized to f32, i.e. the reference's int4_activation = .f32 arithmetic
up to summation order.

RoPE is not taken from that file: its rope() reads x0 = out[:, h, k] as a
numpy view, overwrites out[:, h, k] and then computes the partner element
from the rotated value, so it disagrees with the engine at every position
past 0 (check_tool_rope below shows it). The engine's own rotation,
applyRopeInPlaceOffset (src/forward.zig:353-377: x0, x1 read before either
is written, f32 pow/cos/sin per pair), is restated here instead.

Run in the build container only (it reads /root/reference):
    python tests/golden/make_layer_golden.py
"""
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import layer_case  # noqa: E402

REF = "/root/reference/tools/reference_layer0.py"


def load_reference_primitives():
    spec = importlib.util.spec_from_file_location("reference_layer0", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def rope_engine(x, num_heads, head_dim, theta):
    """forward.zig:353-377 for rows at positions 0..seq-1, in f32."""
    seq = x.shape[0]
    half = head_dim // 2
    k = np.arange(half, dtype=np.float32)
    freq = (np.float32(1.0) / np.power(np.float32(theta),
                                       (np.float32(2.0) * k) / np.float32(head_dim))).astype(np.float32)
    angle = (np.arange(seq, dtype=np.float32)[:, None] * freq[None, :]).astype(np.float32)
    c, s = np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)
    r = x.astype(np.float32).reshape(seq, num_heads, head_dim)
    x0, x1 = r[:, :, :half].copy(), r[:, :, half:].copy()
    out = np.empty_like(r)
    out[:, :, :half] = x0 * c[:, None, :] - x1 * s[:, None, :]
    out[:, :, half:] = x0 * s[:, None, :] + x1 * c[:, None, :]
    return out.reshape(seq, num_heads * head_dim)


def check_tool_rope(ref):
    """The tool's rope() against the engine's rotation on one pair at
    position 1 (returns both; they differ in the second element)."""
    x = np.zeros((2, 4), np.float32)
    x[1] = [1.0, 2.0, 3.0, 4.0]
    return ref.rope(x, 1, 4, 10000.0)[1], rope_engine(x, 1, 4, 10000.0)[1]


def compose(ref, dense, x, cfg):
    """reference_layer0.py main() :107-170 for rows 0..T-1 at positions 0..T-1."""
    eps, theta = cfg["rms_eps"], cfg["rope_theta"]
    n_heads, n_kv, hd = cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    dim = cfg["dim"]
    h_norm = ref.rmsnorm(x, dense["input_norm"], eps)
    q = h_norm @ dense["q"].T + dense["bq"]
    k = h_norm @ dense["k"].T + dense["bk"]
    v = h_norm @ dense["v"].T + dense["bv"]
    q = rope_engine(q, n_heads, hd, theta)
    k = rope_engine(k, n_kv, hd, theta)
    q_r = q.reshape(q.shape[0], n_heads, hd)
    k_r = k.reshape(k.shape[0], n_kv, hd)
    v_r = v.reshape(v.shape[0], n_kv, hd)
    group = n_heads // n_kv
    seq = q.shape[0]
    attn_out = np.zeros((seq, dim), dtype=np.float32)
    scale = 1.0 / np.sqrt(hd)
    for h in range(n_heads):
        kv_h = h // group
        for i in range(seq):
            scores = (q_r[i, h] @ k_r[:i + 1, kv_h].T) * scale
            probs = ref.softmax(scores)
            attn_out[i, h * hd:(h + 1) * hd] = probs @ v_r[:i + 1, kv_h]
    h = x + attn_out @ dense["o"].T
    mlp_norm = ref.rmsnorm(h, dense["post_attn_norm"], eps)
    gate = ref.silu(mlp_norm @ dense["gate"].T) * (mlp_norm @ dense["up"].T)
    out = h + gate @ dense["down"].T
    return out.astype(np.float32), attn_out


def main():
    ref = load_reference_primitives()
    tool, engine = check_tool_rope(ref)
    print("tool rope  ", tool, "\nengine rope", engine)
    _, dense, x = layer_case.make()
    out, attn_out = compose(ref, dense, x, layer_case.CFG)
    path = os.path.join(HERE, "layer_qwen05b.npz")
    np.savez_compressed(path, seed=np.uint64(layer_case.SEED), T=np.int32(layer_case.T),
                        out=out, attn_out=attn_out)
    print("wrote", path, out.shape, float(np.abs(out).max()))


if __name__ == "__main__":
    main()
