"""Python binding of the MI355X Qwen2.5 decode engine (libcuqwen.so, C ABI in
include/cuqwen.h).

The reference (talhatahir-10xe/CuQwen) exposes C++ free functions over raw
device pointers; this module mirrors them for Python callers and tests:

    load_weights(path)              include/load_weights.h:57
    free_weights(weights)           include/load_weights.h:60
    malloc_qwen_state(cfg, weights) include/model.cuh:48
    free_qwen_state(state)          include/model.cuh:49
    qwen_forward(token, pos, cfg, state, weights, history)   include/model.cuh:51-60

plus the op-level `launch_*` family through `lib` (ctypes).  Every call
raises CuQwenError on a non-zero status.  There is no CPU fallback: if the
library is not built, importing the binding raises.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcuqwen.so")

QUANT_FP16, QUANT_INT8, QUANT_INT4 = 0, 1, 2
LMHEAD_FP16, LMHEAD_INT8 = 0, 1
QUANT_NAMES = {"fp16": QUANT_FP16, "int8": QUANT_INT8, "int4": QUANT_INT4}

STATUS = {0: "OK", 1: "EINVAL", 2: "EIO", 3: "EFORMAT", 4: "EHIP", 5: "ENOMEM", 6: "ERANGE"}


class CuQwenError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code


class Config(ctypes.Structure):
    """cq_config: runtime counterpart of the reference's QwenConfig (include/config.h:52-127)."""

    _fields_ = [
        ("vocab_size", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("intermediate_size", ctypes.c_int32),
        ("n_layers", ctypes.c_int32),
        ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("quant_type", ctypes.c_int32),
        ("lm_head_fmt", ctypes.c_int32),
        ("tied", ctypes.c_int32),
        ("norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
    ]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}

    def replace(self, **kw):
        c = Config()
        ctypes.pointer(c)[0] = self
        for k, v in kw.items():
            setattr(c, k, v)
        return c

    def __repr__(self):
        return f"Config({self.as_dict()})"


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python cuqwen_amd/build.py` (or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    P, I32, U64, SZ, F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_float
    CP = ctypes.POINTER(Config)
    IP = ctypes.POINTER(ctypes.c_int32)
    sig = {
        "cq_last_error": (ctypes.c_char_p, []),
        "cq_config_preset": (I32, [ctypes.c_char_p, I32, CP]),
        "cq_read_header": (I32, [ctypes.c_char_p, CP]),
        "cq_write_synthetic_file": (I32, [ctypes.c_char_p, CP, U64]),
        "cq_load_weights": (I32, [ctypes.c_char_p, CP, CP, ctypes.POINTER(P)]),
        "cq_synth_weights": (I32, [CP, U64, ctypes.POINTER(P)]),
        "cq_free_weights": (I32, [P]),
        "cq_weights_tensor": (I32, [P, ctypes.c_char_p, I32, ctypes.POINTER(P), ctypes.POINTER(SZ)]),
        "cq_weights_wo_rows": (I32, [P, I32, ctypes.POINTER(P), ctypes.POINTER(P)]),
        "cq_state_create": (I32, [CP, P, ctypes.POINTER(P)]),
        "cq_state_create_kv": (I32, [CP, P, I32, ctypes.POINTER(P)]),
        "cq_state_destroy": (I32, [P]),
        "cq_forward": (I32, [P, I32, I32, IP, I32, IP]),
        "cq_forward_ex": (I32, [P, P, I32, I32, IP, I32, P, IP]),
        "cq_decode": (I32, [P, I32, I32, I32, IP, I32, IP]),
        "cq_state_logits": (I32, [P, P]),
        "cq_state_fill_kv": (I32, [P, I32, U64]),
        "cq_state_kv_read": (I32, [P, I32, I32, I32, I32, P]),
        "cq_state_kv_write": (I32, [P, I32, I32, I32, I32, P]),
        "cq_state_last_decode_us": (I32, [P, ctypes.POINTER(ctypes.c_double)]),
        "cq_state_set_attention_mode": (I32, [P, I32]),
        "cq_prefill": (I32, [P, IP, I32, I32, IP]),
        "cq_state_last_prefill_us": (I32, [P, ctypes.POINTER(ctypes.c_double)]),
        "cq_synth_normal": (ctypes.c_uint16, [U64, U64, U64, F]),
        "cq_synth_uniform": (ctypes.c_uint32, [U64, U64, U64, ctypes.c_uint32]),
        "cq_tensor_stream_id": (U64, [I32, I32]),
        "cq_kv_stream_id": (U64, [I32, I32, I32]),
        "cq_quantize": (I32, [I32, P, ctypes.c_int64, ctypes.c_int64, I32, P, P]),
        "cq_device_count": (I32, [IP]),
        "cq_malloc": (I32, [ctypes.POINTER(P), SZ]),
        "cq_free": (I32, [P]),
        "cq_memcpy_h2d": (I32, [P, P, SZ]),
        "cq_memcpy_d2h": (I32, [P, P, SZ]),
        "cq_memset": (I32, [P, ctypes.c_int, SZ]),
        "cq_memcpy_d2d": (I32, [P, P, SZ]),
        "cq_synchronize": (I32, []),
        "cq_embedding_lookup": (I32, [P, P, P, I32, P]),
        "cq_rmsnorm": (I32, [P, P, P, I32, F, P]),
        "cq_gemv": (I32, [I32, I32, P, P, P, P, I32, I32, P]),
        "cq_gemv_add": (I32, [I32, P, P, P, P, I32, I32, P]),
        "cq_fused_attn_block": (I32, [I32, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, P, F, F, P]),
        "cq_fused_mlp_stage1": (I32, [I32, P, P, P, P, P, P, P, I32, I32, F, P]),
        "cq_fused_mlp_stage2": (I32, [I32, P, P, P, P, I32, I32, P]),
        "cq_compute_logits": (I32, [I32, P, P, P, P, I32, I32, P]),
        "cq_apply_repetition_penalty": (I32, [P, P, P, I32, F, P, P]),
        "cq_penalty_workspace_bytes": (SZ, [I32]),
        "cq_argmax": (I32, [P, P, I32, P, P]),
        "cq_argmax_workspace_bytes": (SZ, [I32]),
        "cq_kv_k_offset": (ctypes.c_int64, [I32, I32, I32, I32, I32]),
        "cq_kv8_k_offset": (ctypes.c_int64, [I32, I32, I32, I32, I32]),
        "cq_kv8_v_offset": (ctypes.c_int64, [I32, I32, I32, I32, I32]),
        "cq_kv_v_offset": (ctypes.c_int64, [I32, I32, I32, I32, I32]),
        "cq_kv_cache_store": (I32, [P, P, P, P, P, I32, I32, I32, P]),
        "cq_rope": (I32, [P, P, I32, I32, I32, P, ctypes.c_float, P]),
        "cq_gqa_attention_decode": (I32, [P, P, P, P, P, I32, I32, I32, I32, P, P]),
        "cq_attention_workspace_bytes": (SZ, [I32, I32, I32]),
        "cq_gqa_attention_decode_noalloc": (I32, [P, P, P, P, P, I32, I32, I32, I32, P]),
        "cq_noalloc_scratch_bytes": (SZ, []),
        "cq_kv_cache_store_hm": (I32, [P, P, P, P, P, I32, I32, I32, P]),
        "cq_gqa_attention_decode_hm": (I32, [P, P, P, P, P, I32, I32, I32, I32, P, P, P, P]),
        "cq_gqa_attention_decode_kv8": (I32, [P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, P, P]),
        "cq_gqa_attention_decode_fp8": (I32, [P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, P, P]),
        "cq_dequantize": (I32, [I32, I32, P, P, P, I32, I32, P]),
        "cq_time_gemv": (I32, [I32, I32, I32, ctypes.POINTER(P), ctypes.POINTER(P), P, P, I32, I32, I32,
                               ctypes.POINTER(ctypes.c_double)]),
        "cq_time_stream": (I32, [SZ, I32, ctypes.POINTER(P), I32, ctypes.POINTER(ctypes.c_double)]),
        "cq_time_grid_barrier": (I32, [I32, I32, I32, ctypes.POINTER(ctypes.c_double), IP]),
        "cq_state_profile": (I32, [P, I32, I32, I32, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                   ctypes.POINTER(ctypes.c_double), IP]),
        "cq_tokenizer_load": (I32, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "cq_tokenizer_free": (I32, [P]),
        "cq_tokenizer_encode": (I32, [P, ctypes.c_char_p, SZ, IP, I32, IP]),
        "cq_tokenizer_decode": (I32, [P, IP, I32, ctypes.c_char_p, SZ, ctypes.POINTER(SZ)]),
        "cq_tokenizer_token_id": (I32, [P, ctypes.c_char_p]),
        "cq_tokenizer_vocab_size": (I32, [P]),
        "cq_chat_template": (I32, [ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p), I32, I32,
                                   ctypes.c_char_p, SZ, ctypes.POINTER(SZ)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()
EXPORTED = [
    "cq_last_error", "cq_config_preset", "cq_read_header", "cq_write_synthetic_file", "cq_load_weights",
    "cq_synth_weights", "cq_free_weights", "cq_weights_tensor", "cq_weights_wo_rows", "cq_state_create", "cq_state_destroy",
    "cq_forward", "cq_forward_ex", "cq_decode", "cq_state_logits", "cq_state_fill_kv", "cq_state_kv_read", "cq_state_kv_write",
    "cq_prefill", "cq_state_last_prefill_us", "cq_state_create_kv", "cq_gqa_attention_decode_kv8",
    "cq_gqa_attention_decode_fp8",
    "cq_state_last_decode_us", "cq_state_set_attention_mode", "cq_synth_normal", "cq_synth_uniform", "cq_tensor_stream_id", "cq_kv_stream_id",
    "cq_quantize", "cq_device_count", "cq_malloc", "cq_free", "cq_memcpy_h2d", "cq_memcpy_d2h", "cq_memset", "cq_memcpy_d2d",
    "cq_synchronize", "cq_embedding_lookup", "cq_rmsnorm", "cq_gemv", "cq_gemv_add", "cq_fused_attn_block",
    "cq_fused_mlp_stage1", "cq_fused_mlp_stage2", "cq_compute_logits", "cq_apply_repetition_penalty",
    "cq_penalty_workspace_bytes", "cq_argmax", "cq_argmax_workspace_bytes", "cq_kv_k_offset", "cq_kv_v_offset",
    "cq_kv8_k_offset", "cq_kv8_v_offset",
    "cq_kv_cache_store", "cq_rope", "cq_gqa_attention_decode", "cq_attention_workspace_bytes", "cq_dequantize",
    "cq_kv_cache_store_hm", "cq_gqa_attention_decode_hm", "cq_gqa_attention_decode_noalloc",
    "cq_noalloc_scratch_bytes",
    "cq_time_gemv", "cq_time_stream", "cq_time_grid_barrier", "cq_state_profile", "cq_tokenizer_load", "cq_tokenizer_free", "cq_tokenizer_encode",
    "cq_tokenizer_decode", "cq_tokenizer_token_id", "cq_tokenizer_vocab_size", "cq_chat_template",
]


def check(rc):
    if rc != 0:
        raise CuQwenError(rc, lib.cq_last_error().decode(errors="replace"))
    return rc


KV_FP16, KV_INT8, KV_FP8 = 0, 1, 2
ATTN_SPLIT, ATTN_WHOLE_CONTEXT = 0, 1


def preset(model, quant="int8"):
    q = QUANT_NAMES[quant] if isinstance(quant, str) else int(quant)
    c = Config()
    check(lib.cq_config_preset(model.encode(), q, ctypes.byref(c)))
    return c


def read_header(path):
    c = Config()
    check(lib.cq_read_header(os.fsencode(path), ctypes.byref(c)))
    return c


def write_synthetic_file(path, cfg, seed):
    check(lib.cq_write_synthetic_file(os.fsencode(path), ctypes.byref(cfg), seed))


def quantize(quant, w_fp16, group=128):
    """Host quantizer (export_weights.py:123-205) -> (q bytes, fp16 scales)."""
    w = np.ascontiguousarray(w_fp16, dtype=np.float16)
    rows, cols = w.shape
    q = np.zeros((rows, cols // 2 if quant == QUANT_INT4 else cols), dtype=np.uint8)
    ng = cols // group if group else 1
    s = np.zeros((rows, ng), dtype=np.float16)
    check(lib.cq_quantize(quant, w.ctypes.data, rows, cols, group, q.ctypes.data, s.ctypes.data))
    return q, s


def synth_normal_host(seed, stream, n, sigma=1.0, start=0):
    out = np.empty(n, dtype=np.uint16)
    for i in range(n):
        out[i] = lib.cq_synth_normal(seed, stream, start + i, sigma)
    return out.view(np.float16)


# ----------------------------------------------------------- device memory
class DeviceBuffer:
    """Owned device allocation (hipMalloc through the library)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        check(lib.cq_malloc(ctypes.byref(self.ptr), max(self.nbytes, 1)))

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes)
        if arr.nbytes:
            check(lib.cq_memcpy_h2d(b.ptr, arr.ctypes.data, arr.nbytes))
        return b

    def zero(self):
        check(lib.cq_memset(self.ptr, 0, self.nbytes))
        return self

    def to_array(self, dtype, shape=None):
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize
        out = np.empty(n, dtype=dtype)
        if n:
            check(lib.cq_memcpy_d2h(out.ctypes.data, self.ptr, n * dtype.itemsize))
        return out.reshape(shape) if shape is not None else out

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(lib.cq_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes))

    @property
    def value(self):
        return self.ptr.value

    @property
    def _as_parameter_(self):
        return self.ptr

    def free(self):
        if self.ptr:
            # kernels queued on this memory must finish before it is released
            lib.cq_synchronize()
            lib.cq_free(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize():
    check(lib.cq_synchronize())


def device_count():
    n = ctypes.c_int32(0)
    check(lib.cq_device_count(ctypes.byref(n)))
    return n.value


# ------------------------------------------------------------ model level
class Weights:
    """Device weights (QwenWeights, include/load_weights.h:42-54)."""

    def __init__(self, handle, cfg):
        self.handle = handle
        self.cfg = cfg

    def tensor(self, name, layer=-1):
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        check(lib.cq_weights_tensor(self.handle, name.encode(), layer, ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value

    def free(self):
        if self.handle:
            check(lib.cq_free_weights(self.handle))
            self.handle = None


def load_weights(path, expect=None):
    """load_weights() (src/load_weights.cpp:36-165): returns (cfg, Weights)."""
    cfg = Config()
    h = ctypes.c_void_p()
    check(lib.cq_load_weights(os.fsencode(path), ctypes.byref(expect) if expect is not None else None,
                              ctypes.byref(cfg), ctypes.byref(h)))
    return cfg, Weights(h, cfg)


def synth_weights(cfg, seed):
    h = ctypes.c_void_p()
    check(lib.cq_synth_weights(ctypes.byref(cfg), seed, ctypes.byref(h)))
    return Weights(h, cfg)


def free_weights(weights, cfg=None):
    weights.free()


class State:
    """Decode state (QwenState, include/model.cuh:9-46)."""

    def __init__(self, cfg, weights=None, kv_dtype=0):
        """kv_dtype: KV_FP16 (the reference's cache), KV_INT8 or KV_FP8 (E4M3).
        weights may be None (the reference's two-argument malloc_qwen_state):
        the first forward() that passes weights binds them."""
        self.cfg = cfg
        self.weights = weights
        self.kv_dtype = kv_dtype
        self.handle = ctypes.c_void_p()
        check(lib.cq_state_create_kv(ctypes.byref(cfg), weights.handle if weights is not None else None,
                                     int(kv_dtype), ctypes.byref(self.handle)))

    def forward(self, token, pos, history=None, weights=None, stream=None):
        """One synchronous step; `weights` binds (or switches) the weight set,
        `stream` (a hipStream_t as int / c_void_p) runs the step there."""
        hist = np.ascontiguousarray(history if history is not None else [], dtype=np.int32)
        out = ctypes.c_int32(-1)
        check(lib.cq_forward_ex(self.handle, weights.handle if weights is not None else None, int(token), int(pos),
                                hist.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)) if hist.size else None,
                                int(hist.size), stream, ctypes.byref(out)))
        if weights is not None:
            self.weights = weights
        return out.value

    def decode(self, token, pos0, n_steps, history=None):
        hist = np.ascontiguousarray(history if history is not None else [], dtype=np.int32)
        out = np.zeros(n_steps, dtype=np.int32)
        check(lib.cq_decode(self.handle, int(token), int(pos0), int(n_steps),
                            hist.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)) if hist.size else None,
                            int(hist.size), out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))))
        return out

    def prefill(self, tokens, pos0=0):
        """Prompt tokens at positions pos0..: KV cache filled, returns the
        greedy id after the last one (src/main.cu:87-92 semantics)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = ctypes.c_int32(-1)
        check(lib.cq_prefill(self.handle, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), int(t.size), int(pos0),
                             ctypes.byref(out)))
        return out.value

    def last_prefill_us(self):
        us = ctypes.c_double()
        check(lib.cq_state_last_prefill_us(self.handle, ctypes.byref(us)))
        return us.value

    def last_decode_us(self):
        us = ctypes.c_double()
        check(lib.cq_state_last_decode_us(self.handle, ctypes.byref(us)))
        return us.value

    def set_attention_mode(self, mode):
        """ATTN_SPLIT (default) or ATTN_WHOLE_CONTEXT (cq_state_set_attention_mode)."""
        check(lib.cq_state_set_attention_mode(self.handle, mode))

    def logits(self):
        out = np.zeros(self.cfg.vocab_size, dtype=np.uint16)
        check(lib.cq_state_logits(self.handle, out.ctypes.data))
        return out.view(np.float16)

    def fill_kv(self, n_pos, seed):
        check(lib.cq_state_fill_kv(self.handle, int(n_pos), seed))

    def kv_read(self, layer, kv_head, kind, n_pos):
        out = np.zeros((n_pos, self.cfg.head_dim), dtype=np.uint16)
        check(lib.cq_state_kv_read(self.handle, layer, kv_head, kind, n_pos, out.ctypes.data))
        return out.view(np.float16)

    def kv_write(self, layer, kv_head, kind, arr):
        a = np.ascontiguousarray(arr, dtype=np.float16).view(np.uint16)
        check(lib.cq_state_kv_write(self.handle, layer, kv_head, kind, a.shape[0], a.ctypes.data))

    def profile(self, pos, iters=3, max_kernels=16):
        names = ctypes.create_string_buffer(32 * max_kernels)
        us = (ctypes.c_double * max_kernels)()
        by = (ctypes.c_double * max_kernels)()
        n = ctypes.c_int32()
        check(lib.cq_state_profile(self.handle, pos, iters, max_kernels, names, us, by, ctypes.byref(n)))
        res = []
        for i in range(n.value):
            nm = names.raw[32 * i:32 * (i + 1)].split(b"\0", 1)[0].decode()
            res.append({"kernel": nm, "us": us[i], "bytes": by[i], "GBps": by[i] / us[i] / 1e3 if us[i] else 0.0})
        return res

    def free(self):
        if self.handle:
            check(lib.cq_state_destroy(self.handle))
            self.handle = None


def malloc_qwen_state(cfg, weights=None):
    """malloc_qwen_state(config, state) (include/model.cuh:48): weights are
    optional here and bound by the first qwen_forward."""
    return State(cfg, weights)


def free_qwen_state(state):
    state.free()


def qwen_forward(token, pos, cfg, state, weights, history=None, stream=None):
    """qwen_forward() (src/model.cu:183-223): one synchronous decode step -> sampled id."""
    return state.forward(token, pos, history, weights=weights, stream=stream)


# ------------------------------------------------------------- tokenizer
class Tokenizer:
    """QwenTokenizer (include/tokenizer.h:18-41) over the C ABI: the
    exporter's qwen25_bpe_ranks.json in, token ids out and back."""

    def __init__(self, ranks_json_path):
        self.handle = ctypes.c_void_p()
        check(lib.cq_tokenizer_load(os.fsencode(ranks_json_path), ctypes.byref(self.handle)))

    def encode(self, text):
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        cap = len(data) + 16
        while True:
            ids = np.zeros(cap, dtype=np.int32)
            n = ctypes.c_int32()
            rc = lib.cq_tokenizer_encode(self.handle, data, len(data),
                                         ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), cap, ctypes.byref(n))
            if rc == 6 and n.value > cap:   # CQ_ERANGE: grow to the reported size
                cap = n.value
                continue
            check(rc)
            return [int(i) for i in ids[:n.value]]

    def decode_bytes(self, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        need = ctypes.c_size_t()
        cap = max(16, 8 * int(a.size) + 16)
        while True:
            buf = ctypes.create_string_buffer(cap)
            rc = lib.cq_tokenizer_decode(self.handle, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), int(a.size),
                                         buf, cap, ctypes.byref(need))
            if rc == 6 and need.value > cap:
                cap = need.value
                continue
            check(rc)
            return buf.raw[:need.value]

    def decode(self, ids):
        """decode() (src/tokenizer.cpp:203-209): text of the ids (invalid
        UTF-8 from a partial multi-byte character is replaced)."""
        return self.decode_bytes(ids).decode("utf-8", errors="replace")

    def token_id(self, token):
        return int(lib.cq_tokenizer_token_id(self.handle, token.encode("utf-8")))

    def vocab_size(self):
        return int(lib.cq_tokenizer_vocab_size(self.handle))

    @staticmethod
    def apply_chat_template(messages, add_generation_prompt=True):
        """apply_chat_template (src/tokenizer.cpp:98-105); messages are
        (role, content) pairs or {"role", "content"} dicts."""
        pairs = [(m["role"], m["content"]) if isinstance(m, dict) else tuple(m) for m in messages]
        n = len(pairs)
        roles = (ctypes.c_char_p * max(n, 1))(*[r.encode("utf-8") for r, _ in pairs])
        contents = (ctypes.c_char_p * max(n, 1))(*[c.encode("utf-8") for _, c in pairs])
        need = ctypes.c_size_t()
        rc = lib.cq_chat_template(roles, contents, n, int(bool(add_generation_prompt)), None, 0, ctypes.byref(need))
        if rc not in (0, 6):
            check(rc)
        buf = ctypes.create_string_buffer(max(1, need.value))
        check(lib.cq_chat_template(roles, contents, n, int(bool(add_generation_prompt)), buf, need.value,
                                   ctypes.byref(need)))
        return buf.raw[:need.value].decode("utf-8")

    def free(self):
        if self.handle:
            check(lib.cq_tokenizer_free(self.handle))
            self.handle = None


class ChatSession:
    """The turn logic of the reference's chat loop (src/main.cu:40-126) as a
    library object: the first turn sends the whole templated conversation,
    later turns only the new user turn; the prompt is prefilled (batched here,
    one decode step per token there), then greedy decode with the turn's
    generated ids as the repetition-penalty history until <|endoftext|> or
    <|im_end|> (neither is fed back) or the context limit (max_seq_len - 2)."""

    def __init__(self, state, tokenizer, eos_id=151643, im_end_id=151645):
        self.state = state
        self.tok = tokenizer
        self.eos_id = eos_id
        self.im_end_id = im_end_id
        self.history = []
        self.pos = 0

    def reply(self, user_text, max_new_tokens=None, on_token=None):
        limit = self.state.cfg.max_seq_len - 2
        self.history.append(("user", user_text))
        turn = self.history if len(self.history) == 1 else [("user", user_text)]
        prompt = self.tok.encode(self.tok.apply_chat_template(turn, True))
        if self.pos + len(prompt) >= limit:
            raise CuQwenError(6, "prompt too long for the remaining context")
        nxt = self.state.prefill(prompt, self.pos)
        self.pos += len(prompt)
        generated = []
        while nxt not in (self.eos_id, self.im_end_id) and self.pos < limit:
            if max_new_tokens is not None and len(generated) >= max_new_tokens:
                break
            generated.append(nxt)
            if on_token:
                on_token(nxt)
            nxt = self.state.forward(nxt, self.pos, generated)
            self.pos += 1
        text = self.tok.decode(generated)
        self.history.append(("assistant", text))
        return text, generated
