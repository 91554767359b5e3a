"""The Qwen2.5-7B-shaped test model of q7b_*.npz, shared by
make_7b_golden.py (which writes the fixtures) and the GPU tests.

Weights come from the product's synthetic generator (glacier_hip_synth_*),
then two changes make greedy decoding discriminative: RMSNorm weights are
1 + N(0, 0.02), and in every INT4 tensor the code 15 is replaced by 7, so the
decoded values (u - 7) are symmetric around 0 with mean 0. With codes uniform
on 0..15 the decoded values have mean +0.5, every projection carries the same
rank-one component, and the 28-layer model emits one token whatever the
prompt. The kernels' decode is unchanged (u - 7, low nibble first)."""
import numpy as np

Q7B = dict(num_layers=28, dim=3584, hidden_dim=18944, num_heads=28, num_kv_heads=4, head_dim=128,
           vocab_size=152064, group_size=32, rms_eps=1e-6, rope_theta=1e6)
SEED = 0x474C4143
PROMPT_ID = 0x37425052
PROMPT_LEN = 16
MAX_NEW = 32
STEPS = [0, 1, 16, 31]
# the shallow variant: the same geometry with two layers, 128 greedy tokens
SHALLOW_LAYERS = 2
SHALLOW_MAX_NEW = 128


def _symmetric_lut():
    b = np.arange(256, dtype=np.uint16)
    lo, hi = b & 0x0F, b >> 4
    lo = np.where(lo == 15, 7, lo)
    hi = np.where(hi == 15, 7, hi)
    return (lo | (hi << 4)).astype(np.uint8)


_LUT = _symmetric_lut()


def _symmetric(packed):
    """Every nibble 15 becomes 7 (both nibbles of each byte)."""
    return np.take(_LUT, packed)


def shallow_cfg():
    return dict(Q7B, num_layers=SHALLOW_LAYERS)


def symmetric_codes(host):
    """Every INT4 tensor of a host model with nibble 15 replaced by 7."""
    for L in host["layers"]:
        for k in [k for k in L if k.startswith("w_")]:
            L[k] = _symmetric(L[k])
    host["lm_head"] = _symmetric(host["lm_head"])
    return host


def make_host(gh, cfg=Q7B):
    host = gh.random_model_host(cfg, SEED)
    for L in host["layers"]:
        L["input_norm"] = (L["input_norm"] + 1.0).astype(np.float32)
        L["post_attn_norm"] = (L["post_attn_norm"] + 1.0).astype(np.float32)
    host["final_norm"] = (host["final_norm"] + 1.0).astype(np.float32)
    return symmetric_codes(host)


def prompt(gh):
    return gh.synth_tokens(SEED, PROMPT_ID, Q7B["vocab_size"], PROMPT_LEN)
