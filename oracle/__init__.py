"""ctypes binding of the CPU oracle (oracle/glacier_oracle.c).

TEST INFRASTRUCTURE ONLY. The oracle restates the reference CPU path and is
used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
the checker; the product never imports it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libglacier_oracle.so")

OK, SHAPE_MISMATCH, BAD_GROUP_SIZE, TRUNCATED, INVALID_MASK, ELIGIBLE_NAN, NO_MEMORY = range(7)


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


_lib = None
_P = C.c_void_p


class Int4Weight(C.Structure):
    _fields_ = [("packed", _P), ("scales", _P)]


class Layer(C.Structure):
    _fields_ = [("input_norm", _P), ("post_attn_norm", _P)] + \
        [(n, Int4Weight) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")] + \
        [("bq", _P), ("bk", _P), ("bv", _P)]


class Model(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("num_layers", "dim", "hidden_dim", "num_heads",
                                          "num_kv_heads", "head_dim", "vocab_size", "group_size")] + \
        [("rms_eps", C.c_float), ("rope_theta", C.c_float), ("token_embedding", _P),
         ("final_norm", _P), ("lm_head", Int4Weight), ("layers", _P), ("kv_fp16", C.c_uint32),
         ("int4_activation_f32", C.c_uint32)]


class Ledger(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "page_count_capacity", "page_elements", "page_payload_bytes", "tensor_capacity_bytes",
        "page_map_bytes", "allocation_capacity_bytes", "contiguous_counterfactual_bytes",
        "capacity_reclaimed_bytes", "capacity_overhead_bytes", "padded_positions")]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        sz = C.c_size_t
        sig = {
            "go_set_threads": (None, [C.c_int]),
            "go_int4_quantize": (C.c_int, [_P, sz, C.c_uint32, _P, _P]),
            "go_int4_dequantize": (C.c_int, [_P, sz, _P, sz, C.c_uint32, sz, _P]),
            "go_f32_to_f16": (C.c_uint16, [C.c_float]),
            "go_f16_to_f32": (C.c_float, [C.c_uint16]),
            "go_linear_int4_f32": (C.c_int, [_P, sz, _P, _P, _P, _P, sz, sz, sz]),
            "go_q8_quantize": (C.c_int, [_P, sz, sz, _P, _P]),
            "go_linear_int4_q8": (C.c_int, [_P, sz, _P, _P, _P, _P, sz, sz, sz]),
            "go_linear_int4_weight_q8": (C.c_int, [_P, sz, _P, _P, _P, _P, sz, sz, sz]),
            "go_rmsnorm": (C.c_int, [_P, sz, sz, _P, C.c_float, _P]),
            "go_silu_mul": (None, [_P, _P, _P, sz]),
            "go_rope_table": (None, [sz, sz, C.c_float, _P, _P]),
            "go_rope_apply": (None, [_P, _P, sz, _P, sz, sz, sz]),
            "go_rope_apply_direct": (None, [_P, sz, sz, sz, C.c_float]),
            "go_attention": (C.c_int, [_P, sz, _P, _P, sz, _P, sz, sz, sz]),
            "go_attention_paged": (C.c_int, [_P, sz, _P, C.c_int, _P, sz, sz, sz, _P, sz, sz, sz]),
            "go_argmax": (sz, [_P, sz]),
            "go_argmax_eligible": (C.c_int, [_P, sz, _P, sz, C.POINTER(sz), C.POINTER(sz)]),
            "go_generate": (C.c_int, [C.POINTER(Model), _P, sz, sz, _P, _P, sz, _P, _P, _P]),
            "go_generate_forced": (C.c_int, [C.POINTER(Model), _P, sz, sz, _P, _P, _P, sz, _P]),
            "go_forward_layer": (C.c_int, [C.POINTER(Model), sz, _P, _P, _P, sz, _P, _P, _P]),
            "go_sha256": (None, [_P, sz, _P]),
            "go_paged_capacity_ledger": (C.c_int, [C.c_uint64] * 3 + [C.POINTER(Ledger)]),
            "go_paged_empty_ownership_digest": (None, [C.c_uint64] * 4 + [_P]),
            "go_paged_append_ownership_digest": (None, [_P] + [C.c_uint64] * 3 + [_P]),
            "go_token_sequence_sha256": (None, [_P, sz, _P]),
            "go_logical_kv_sha256": (None, [_P, _P, sz, sz, sz, sz, _P]),
            "go_xoshiro256_init": (None, [C.c_uint64, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def set_threads(n):
    lib().go_set_threads(int(n))


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def int4_quantize(src, group):
    src = f32(src)
    n = src.size
    packed = np.zeros((n + 1) // 2, dtype=np.uint8)
    scales = np.zeros(-(-n // group), dtype=np.float32)
    rc = lib().go_int4_quantize(_p(src), n, group, _p(packed), _p(scales))
    return rc, packed, scales


def int4_dequantize(packed, scales, group, n):
    out = np.zeros(n, dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = f32(scales)
    rc = lib().go_int4_dequantize(_p(packed), packed.size, _p(scales), scales.size, group, n, _p(out))
    return rc, out


def linear_int4_f32(x, packed, scales, out_f, in_f, group, bias=None):
    x = f32(x).reshape(-1, in_f)
    out = np.zeros((x.shape[0], out_f), dtype=np.float32)
    b = None if bias is None else f32(bias)
    rc = lib().go_linear_int4_f32(_p(x), x.shape[0], _p(np.ascontiguousarray(packed)), _p(f32(scales)),
                                  _p(b), _p(out), out_f, in_f, group)
    assert rc == OK, rc
    return out


def linear_int4_q8(x, packed, scales, out_f, in_f, group, bias=None):
    x = f32(x).reshape(-1, in_f)
    out = np.zeros((x.shape[0], out_f), dtype=np.float32)
    b = None if bias is None else f32(bias)
    rc = lib().go_linear_int4_q8(_p(x), x.shape[0], _p(np.ascontiguousarray(packed)), _p(f32(scales)),
                                 _p(b), _p(out), out_f, in_f, group)
    assert rc == OK, rc
    return out


def q8_quantize(x, group):
    x = f32(x)
    q = np.zeros(x.size, dtype=np.int8)
    s = np.zeros(-(-x.size // group), dtype=np.float32)
    rc = lib().go_q8_quantize(_p(x), x.size, group, _p(q), _p(s))
    assert rc == OK
    return q, s


def rmsnorm(x, w, eps):
    x = f32(x)
    rows = x.reshape(-1, x.shape[-1])
    out = np.zeros_like(rows)
    lib().go_rmsnorm(_p(rows), rows.shape[0], rows.shape[1], _p(f32(w)), eps, _p(out))
    return out.reshape(x.shape)


def silu_mul(g, u):
    g, u = f32(g), f32(u)
    out = np.zeros_like(g)
    lib().go_silu_mul(_p(g), _p(u), _p(out), g.size)
    return out


def rope_table(positions, head_dim, theta):
    half = head_dim // 2
    cs = np.zeros(positions * half, dtype=np.float32)
    sn = np.zeros(positions * half, dtype=np.float32)
    lib().go_rope_table(positions, head_dim, theta, _p(cs), _p(sn))
    return cs, sn


def rope_apply_direct(row, pos, heads, head_dim, theta):
    r = f32(row).copy()
    lib().go_rope_apply_direct(_p(r), pos, heads, head_dim, theta)
    return r


def attention(q, k, v, num_heads, num_kv_heads, head_dim):
    q, k, v = f32(q), f32(k), f32(v)
    q_dim = num_heads * head_dim
    q_seq = q.size // q_dim
    kv_seq = k.size // (num_kv_heads * head_dim)
    out = np.zeros(q_seq * q_dim, dtype=np.float32)
    rc = lib().go_attention(_p(q), q_seq, _p(k), _p(v), kv_seq, _p(out), num_heads, num_kv_heads, head_dim)
    assert rc == OK, rc
    return out.reshape(q_seq, q_dim)


def attention_paged(q, pool, kv_fp16, page_table, kv_seq, layer, num_layers, num_heads,
                    num_kv_heads, head_dim):
    q = f32(q)
    q_dim = num_heads * head_dim
    q_seq = q.size // q_dim
    pt = np.ascontiguousarray(page_table, dtype=np.int32)
    pool = np.ascontiguousarray(pool)
    out = np.zeros(q_seq * q_dim, dtype=np.float32)
    rc = lib().go_attention_paged(_p(q), q_seq, _p(pool), 1 if kv_fp16 else 0, _p(pt), kv_seq, layer,
                                  num_layers, _p(out), num_heads, num_kv_heads, head_dim)
    assert rc == OK, rc
    return out.reshape(q_seq, q_dim)


def argmax(v):
    v = f32(v)
    return int(lib().go_argmax(_p(v), v.size))


def argmax_eligible(logits, words):
    logits = f32(logits)
    words = np.ascontiguousarray(words, dtype=np.uint64)
    idx, rows = C.c_size_t(), C.c_size_t()
    rc = lib().go_argmax_eligible(_p(logits), logits.size, _p(words), words.size,
                                  C.byref(idx), C.byref(rows))
    return rc, idx.value, rows.value


def sha256(data):
    b = np.frombuffer(bytes(data), dtype=np.uint8) if len(data) else np.zeros(1, np.uint8)
    out = np.zeros(32, dtype=np.uint8)
    lib().go_sha256(_p(b), len(data), _p(out))
    return out.tobytes()


def capacity_ledger(num_layers, dim, max_seq):
    led = Ledger()
    rc = lib().go_paged_capacity_ledger(num_layers, dim, max_seq, C.byref(led))
    return rc, {n: getattr(led, n) for n, _ in Ledger._fields_}


def empty_ownership_digest(inst, num_layers, dim, max_seq):
    out = np.zeros(32, dtype=np.uint8)
    lib().go_paged_empty_ownership_digest(inst, num_layers, dim, max_seq, _p(out))
    return out.tobytes()


def append_ownership_digest(before, inst, page, gen):
    b = np.frombuffer(before, dtype=np.uint8).copy()
    out = np.zeros(32, dtype=np.uint8)
    lib().go_paged_append_ownership_digest(_p(b), inst, page, gen, _p(out))
    return out.tobytes()


def logical_kv_sha256(k, v, positions):
    """logicalKvPrefixSha256 of the first `positions` rows of k, v [L][max_seq][kv_dim]."""
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    assert k.shape == v.shape and k.ndim == 3 and positions <= k.shape[1]
    out = np.zeros(32, dtype=np.uint8)
    lib().go_logical_kv_sha256(_p(k), _p(v), k.shape[0], k.shape[1], k.shape[2], positions,
                               _p(out))
    return out.tobytes()


def token_sequence_sha256(tokens):
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = np.zeros(32, dtype=np.uint8)
    lib().go_token_sequence_sha256(_p(t) if t.size else None, t.size, _p(out))
    return out.tobytes()


def xoshiro256_init(seed):
    s = np.zeros(4, dtype=np.uint64)
    lib().go_xoshiro256_init(seed, _p(s))
    return [int(v) for v in s]


class OracleModel:
    """Keeps the numpy tensors alive while the C model struct points at them."""

    def __init__(self, cfg, host, kv_fp16=False, act_f32=False):
        self.cfg = cfg
        self.host = host
        self._keep = []
        layers = (Layer * cfg["num_layers"])()
        keep = self._keep.append

        def w(packed, scales):
            packed = np.ascontiguousarray(packed, dtype=np.uint8)
            scales = f32(scales)
            keep(packed)
            keep(scales)
            return Int4Weight(_p(packed), _p(scales))

        def arr(a):
            if a is None:
                return None
            a = f32(a)
            keep(a)
            return _p(a)

        for i, L in enumerate(host["layers"]):
            layers[i] = Layer(arr(L["input_norm"]), arr(L["post_attn_norm"]),
                              w(L["w_q"], L["s_q"]), w(L["w_k"], L["s_k"]), w(L["w_v"], L["s_v"]),
                              w(L["w_o"], L["s_o"]), w(L["w_gate"], L["s_gate"]),
                              w(L["w_up"], L["s_up"]), w(L["w_down"], L["s_down"]),
                              arr(L.get("bq")), arr(L.get("bk")), arr(L.get("bv")))
        self._layers = layers
        self.m = Model(cfg["num_layers"], cfg["dim"], cfg["hidden_dim"], cfg["num_heads"],
                       cfg["num_kv_heads"], cfg["head_dim"], cfg["vocab_size"], cfg["group_size"],
                       cfg["rms_eps"], cfg["rope_theta"], arr(host["embedding"]),
                       arr(host["final_norm"]), w(host["lm_head"], host["lm_head_scales"]),
                       C.cast(layers, _P), 1 if kv_fp16 else 0, 1 if act_f32 else 0)

    def forward_layer(self, li, xs):
        """go_forward_layer over rows xs[t] at positions t = 0..T-1 (token at a
        time over a contiguous f32 KV cache); returns the layer outputs [T, dim]."""
        xs = f32(xs)
        T, D = xs.shape
        kvd = self.cfg["num_kv_heads"] * self.cfg["head_dim"]
        kc = np.zeros((T, kvd), np.float32)
        vc = np.zeros((T, kvd), np.float32)
        cs, sn = rope_table(T, self.cfg["head_dim"], self.cfg["rope_theta"])
        out = np.zeros_like(xs)
        for t in range(T):
            rc = lib().go_forward_layer(C.byref(self.m), li, _p(xs[t]), _p(kc), _p(vc), t,
                                        _p(cs), _p(sn), _p(out[t]))
            assert rc == OK, rc
        return out

    def forward_layer_at(self, li, x, k_hist, v_hist):
        """go_forward_layer for one token at position p = len(k_hist) over a
        given K/V history of this layer ([p, kv_dim] rows, e.g. read back from
        a device cache); returns (layer output, the K row, the V row)."""
        x = f32(x)
        p = len(k_hist)
        kvd = self.cfg["num_kv_heads"] * self.cfg["head_dim"]
        kc = np.zeros((p + 1, kvd), np.float32)
        vc = np.zeros((p + 1, kvd), np.float32)
        kc[:p], vc[:p] = k_hist, v_hist
        cs, sn = rope_table(p + 1, self.cfg["head_dim"], self.cfg["rope_theta"])
        out = np.zeros_like(x)
        rc = lib().go_forward_layer(C.byref(self.m), li, _p(x), _p(kc), _p(vc), p, _p(cs),
                                    _p(sn), _p(out))
        assert rc == OK, rc
        return out, kc[p].copy(), vc[p].copy()

    def generate_forced(self, prompt, forced, logits_steps=()):
        """Greedy argmax of every step with step s >= 1 fed forced[s - 1];
        returns (argmax tokens, logits at logits_steps)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        forced = np.ascontiguousarray(forced, dtype=np.uint32)
        max_new = forced.size + 1
        toks = np.zeros(max_new, dtype=np.uint32)
        steps = np.ascontiguousarray(list(logits_steps) or [-1], dtype=np.int32)
        logits = np.zeros((max(len(logits_steps), 1), self.cfg["vocab_size"]), dtype=np.float32)
        rc = lib().go_generate_forced(C.byref(self.m), _p(prompt), prompt.size, max_new,
                                      _p(forced), _p(toks), _p(steps), len(logits_steps),
                                      _p(logits))
        assert rc == OK, rc
        return toks, logits

    def generate(self, prompt, max_new, logits_steps=()):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        toks = np.zeros(max_new, dtype=np.uint32)
        steps = np.ascontiguousarray(list(logits_steps) or [-1], dtype=np.int32)
        V = self.cfg["vocab_size"]
        logits = np.zeros((max(len(logits_steps), 1), V), dtype=np.float32)
        kv = np.zeros(32, dtype=np.uint8)
        out = np.zeros(32, dtype=np.uint8)
        rc = lib().go_generate(C.byref(self.m), _p(prompt), prompt.size, max_new, _p(toks),
                               _p(steps), len(logits_steps), _p(logits), _p(kv), _p(out))
        assert rc == OK, rc
        return toks, logits[:len(logits_steps)], kv.tobytes(), out.tobytes()
