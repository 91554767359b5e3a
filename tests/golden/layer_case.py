"""Inputs of the one-layer composition fixture (layer_qwen05b.npz): a
Qwen2.5-0.5B-shaped decoder layer with INT4 group-32 weights (codes u in
0..15 decoding to (u - 7) * scale, low nibble = even element; fp16 scales
from |N(0, 0.02)|), q/k/v biases, unit-centred norms, and T input rows
x ~ N(0, 1), all from numpy's PCG64 with a fixed seed.

Shared by make_layer_golden.py (which writes the fixture) and the test that
checks the oracle against it."""
import numpy as np

CFG = dict(num_layers=1, dim=896, hidden_dim=4864, num_heads=14, num_kv_heads=2, head_dim=64,
           vocab_size=128, group_size=32, rms_eps=1e-6, rope_theta=1e6)
SEED = 0x4C41594552
T = 8


def _int4(rng, out_f, in_f):
    codes = rng.integers(0, 16, size=(out_f, in_f), dtype=np.uint8)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    scales = np.abs(rng.normal(0.0, 0.02, size=(out_f, in_f // 32))).astype(np.float16)
    scales = scales.astype(np.float32)
    dense = (codes.astype(np.float32) - 7.0) * np.repeat(scales, 32, axis=1)
    return packed, scales.reshape(-1), dense


def make():
    """Returns (layer dict for oracle.OracleModel, dense f32 weights, x[T, dim])."""
    c = CFG
    rng = np.random.default_rng(SEED)
    D, F, kvd = c["dim"], c["hidden_dim"], c["num_kv_heads"] * c["head_dim"]
    layer, dense = {}, {}
    for name, (o, i) in dict(q=(D, D), k=(kvd, D), v=(kvd, D), o=(D, D), gate=(F, D), up=(F, D),
                             down=(D, F)).items():
        p, s, w = _int4(rng, o, i)
        layer["w_" + name], layer["s_" + name], dense[name] = p, s, w
    for b, n in (("bq", D), ("bk", kvd), ("bv", kvd)):
        layer[b] = rng.normal(0.0, 0.1, size=n).astype(np.float32)
        dense[b] = layer[b]
    for nm in ("input_norm", "post_attn_norm"):
        layer[nm] = (1.0 + rng.normal(0.0, 0.02, size=D)).astype(np.float32)
        dense[nm] = layer[nm]
    x = rng.normal(0.0, 1.0, size=(T, D)).astype(np.float32)
    return layer, dense, x
