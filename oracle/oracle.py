"""ctypes wrapper of the scalar host oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker; never by the product.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

# generator tensor kinds (must match the product's stream ids)
K_EMBED, K_FINAL_NORM, K_LM_HEAD, K_IN_NORM, K_WQ, K_BQ, K_WK, K_BK, K_WV, K_BV, K_WO, K_POST_NORM, K_WG, K_WU, K_WD = range(15)


def build():
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    P, I, I64, U64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float
    sig = {
        "or_set_threads": (None, [I]),
        "or_max_threads": (I, []),
        "or_f2h": (ctypes.c_uint16, [F]),
        "or_h2f": (F, [ctypes.c_uint16]),
        "or_gen_half": (ctypes.c_uint16, [U64, U64, U64, F, F]),
        "or_tensor_stream": (U64, [I, I]),
        "or_kv_stream": (U64, [I, I, I]),
        "or_quantize": (None, [I, P, I64, I64, I64, P, P]),
        "or_gemv": (None, [I, P, P, P, P, I64, I64, I64, I]),
        "or_rmsnorm": (None, [P, P, P, I64, F, I]),
        "or_rope": (None, [P, I, I, I, F]),
        "or_attention": (None, [P, P, P, P, I, I, I, I64, I, I, I]),
        "or_argmax": (I, [P, I]),
        "or_quant_row_i8": (None, [P, I, P, P]),
        "or_attention_i8": (None, [P, P, P, P, P, P, I, I, I, I64, I, I, I]),
        "or_attention_kvq": (None, [P, P, P, P, P, P, I, I, I, I64, I, I, I, I]),
        "or_quant_row_f8": (None, [P, I, P, P]),
        "or_e4m3_encode": (None, [P, I64, P]),
        "or_e4m3_decode": (None, [P, I64, P]),
        "or_model_set_kv8": (None, [P, I]),
        "or_model_kv8": (None, [P, I, I, I, I, P, P]),
        "or_penalty": (None, [P, P, I, I, F]),
        "or_model_synth": (P, [P, U64, I]),
        "or_model_load": (P, [ctypes.c_char_p, I]),
        "or_model_free": (None, [P]),
        "or_model_set_nparts": (None, [P, I]),
        "or_model_fill_kv": (None, [P, I, U64]),
        "or_model_forward": (I, [P, I, I, P, I, I]),
        "or_model_logits": (None, [P, P]),
        "or_model_last_times": (None, [P, P]),
        "or_model_kv": (None, [P, I, I, I, I, P]),
        "or_model_tensor": (I64, [P, I, I, I, P]),
    }
    for n, (r, a) in sig.items():
        f = getattr(lib, n)
        f.restype = r
        f.argtypes = a
    return lib


lib = _load()


def _p(a):
    return a.ctypes.data if a is not None else None


def set_threads(n):
    lib.or_set_threads(int(n))


def f2h_bits(values):
    return np.array([lib.or_f2h(float(v)) for v in values], dtype=np.uint16)


def gen_half(seed, stream, n, sigma=1.0, mean=0.0, start=0):
    return np.array([lib.or_gen_half(seed, stream, start + i, sigma, mean) for i in range(n)],
                    dtype=np.uint16).view(np.float16)


def quantize(quant, w, group=128):
    w = np.ascontiguousarray(w, dtype=np.float16)
    rows, cols = w.shape
    q = np.zeros((rows, cols // 2 if quant == 2 else cols), dtype=np.uint8)
    s = np.zeros((rows, cols // group if group else 1), dtype=np.float16)
    lib.or_quantize(quant, _p(w), rows, cols, group, _p(q), _p(s))
    return q, s


def gemv(quant, W, S, x, rows, cols, group=128, mode=0):
    W = np.ascontiguousarray(W)
    x = np.ascontiguousarray(x, dtype=np.float16)
    S = np.ascontiguousarray(S, dtype=np.float16) if S is not None else None
    y = np.zeros(rows, dtype=np.float32)
    lib.or_gemv(quant, _p(W), _p(S), _p(x), _p(y), rows, cols, group, mode)
    return y


def rmsnorm(x, w, eps=1e-6, mode=0):
    x = np.ascontiguousarray(x, dtype=np.float16)
    w = np.ascontiguousarray(w, dtype=np.float16)
    out = np.zeros_like(x)
    lib.or_rmsnorm(_p(x), _p(w), _p(out), x.size, eps, mode)
    return out


def rope(v, n_heads, hd, pos, theta=1e6):
    v = np.ascontiguousarray(v, dtype=np.float16).copy()
    lib.or_rope(_p(v), n_heads, hd, pos, theta)
    return v


def attention(q, K, V, n_heads, n_kv, hd, T, mode=0, nparts=64):
    """K, V: [n_kv][stride][hd] fp16 head-major; keys [0, T)."""
    q = np.ascontiguousarray(q, dtype=np.float16)
    K = np.ascontiguousarray(K, dtype=np.float16)
    V = np.ascontiguousarray(V, dtype=np.float16)
    stride = K.shape[1]
    out = np.zeros(n_heads * hd, dtype=np.float16)
    lib.or_attention(_p(q), _p(K), _p(V), _p(out), n_heads, n_kv, hd, stride, T, mode, nparts)
    return out


def quant_rows_i8(x):
    """int8 KV quantization of each row of x (fp16 [n][hd]): (q int8, s fp32)."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    n, hd = x.shape
    q = np.zeros((n, hd), dtype=np.int8)
    s = np.zeros(n, dtype=np.float32)
    for i in range(n):
        lib.or_quant_row_i8(_p(x[i]), hd, _p(q[i]), _p(s[i:i + 1]))
    return q, s


def attention_i8(q, Kq, Ks, Vq, Vs, n_heads, n_kv, hd, T, mode=0, nparts=64, fmt=1):
    """Attention over a quantized cache: Kq/Vq [n_kv][T][hd] bytes (fmt 1:
    int8, 2: E4M3), Ks/Vs [n_kv][T] fp32."""
    Kq = np.ascontiguousarray(Kq).view(np.int8)
    Vq = np.ascontiguousarray(Vq).view(np.int8)
    Ks, Vs = np.ascontiguousarray(Ks, dtype=np.float32), np.ascontiguousarray(Vs, dtype=np.float32)
    out = np.zeros(n_heads * hd, dtype=np.uint16)
    qq = np.ascontiguousarray(q, dtype=np.float16)
    lib.or_attention_kvq(_p(qq), _p(Kq), _p(Ks), _p(Vq), _p(Vs), _p(out), n_heads, n_kv, hd, Kq.shape[1], T, mode,
                         nparts, fmt)
    return out.view(np.float16)


def quant_rows_f8(x):
    """E4M3 KV quantization of each row of x (fp16 [n][hd]): (q uint8 codes, s fp32)."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    n, hd = x.shape
    q = np.zeros((n, hd), dtype=np.uint8)
    s = np.zeros(n, dtype=np.float32)
    for i in range(n):
        lib.or_quant_row_f8(_p(x[i]), hd, _p(q[i]), _p(s[i:i + 1]))
    return q, s


def quant_rows_kv(x, fmt):
    """Rows quantized in KV format fmt (1 int8, 2 E4M3); codes as uint8."""
    if fmt == 2:
        return quant_rows_f8(x)
    q, s = quant_rows_i8(x)
    return q.view(np.uint8), s


def e4m3_encode(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.shape, dtype=np.uint8)
    lib.or_e4m3_encode(_p(x), x.size, _p(out))
    return out


def e4m3_decode(b):
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.zeros(b.shape, dtype=np.float32)
    lib.or_e4m3_decode(_p(b), b.size, _p(out))
    return out


def kv_decode(codes, fmt):
    """Values of stored cache bytes (before the row scale)."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    return e4m3_decode(codes) if fmt == 2 else codes.view(np.int8).astype(np.float32)


def argmax(logits):
    l = np.ascontiguousarray(logits, dtype=np.float16)
    return lib.or_argmax(_p(l), l.size)


def penalty(logits, hist, pen=1.1):
    l = np.ascontiguousarray(logits, dtype=np.float16).copy()
    h = np.ascontiguousarray(hist, dtype=np.int32)
    lib.or_penalty(_p(l), _p(h), h.size, l.size, pen)
    return l


class Model:
    """Host model for decode parity: synthetic (same generator as the product) or from a weight file."""

    def __init__(self, handle, cfg):
        if not handle:
            raise RuntimeError("oracle: model creation failed")
        self.h = handle
        self.cfg = cfg

    @classmethod
    def synth(cls, cfg, seed, kv_slots):
        c = np.array([cfg.vocab_size, cfg.dim, cfg.intermediate_size, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads,
                      cfg.head_dim, cfg.max_seq_len, cfg.quant_type, cfg.lm_head_fmt, cfg.tied], dtype=np.int32)
        return cls(lib.or_model_synth(_p(c), seed, kv_slots), cfg)

    @classmethod
    def load(cls, path, cfg, kv_slots):
        return cls(lib.or_model_load(os.fsencode(path), kv_slots), cfg)

    def set_nparts(self, n):
        lib.or_model_set_nparts(self.h, n)

    def set_kv8(self, on=True):
        """Quantized KV cache (clears the cache): True / 1 int8, 2 E4M3, 0 fp16."""
        lib.or_model_set_kv8(self.h, int(on))

    def kv8(self, layer, kv_head, kind, n):
        """Raw rows (int8 array; E4M3 codes viewed as int8) and scales."""
        q = np.zeros((n, self.cfg.head_dim), dtype=np.int8)
        s = np.zeros(n, dtype=np.float32)
        lib.or_model_kv8(self.h, layer, kv_head, kind, n, _p(q), _p(s))
        return q, s

    def fill_kv(self, n_pos, seed):
        lib.or_model_fill_kv(self.h, n_pos, seed)

    def forward(self, token, pos, history=None, mode=0):
        h = np.ascontiguousarray(history if history is not None else [], dtype=np.int32)
        r = lib.or_model_forward(self.h, int(token), int(pos), _p(h) if h.size else None, h.size, mode)
        if r < 0:
            raise ValueError("oracle: bad token / pos")
        return r

    def last_times(self):
        """(embedding + layers, head) seconds of the last forward()."""
        t = np.zeros(2, dtype=np.float64)
        lib.or_model_last_times(self.h, _p(t))
        return float(t[0]), float(t[1])

    def logits(self):
        out = np.zeros(self.cfg.vocab_size, dtype=np.uint16)
        lib.or_model_logits(self.h, _p(out))
        return out.view(np.float16)

    def kv(self, layer, kv_head, kind, n):
        out = np.zeros((n, self.cfg.head_dim), dtype=np.uint16)
        lib.or_model_kv(self.h, layer, kv_head, kind, n, _p(out))
        return out.view(np.float16)

    def tensor(self, layer, kind, which=0):
        n = lib.or_model_tensor(self.h, layer, kind, which, None)
        out = np.zeros(n, dtype=np.uint8)
        if n:
            lib.or_model_tensor(self.h, layer, kind, which, _p(out))
        return out

    def __del__(self):
        if getattr(self, "h", None) and lib is not None:
            lib.or_model_free(self.h)
            self.h = None
