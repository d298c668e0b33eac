"""The reference's op-level API through include/cuqwen_compat.hpp on the GPU.

tests/compat/kernel_caller.cpp makes the calls benchmark/kernel_profile.cu:
66-85 makes (launch_rmsnorm, launch_fused_attn_block, launch_kv_cache_store,
launch_gqa_attention_decode, launch_gemv_add_fp16, launch_fused_mlp_stage1/2,
launch_embedding_lookup, launch_compute_logits, launch_apply_repetition_penalty,
launch_argmax, plus launch_compute_logits_int8), with its buffers sized from
QwenConfig, on seeded data, and writes every input and output; each op is
checked here against the oracle on the inputs it saw.  Bars: bit-exact for
the embedding row, the KV-cache placement, the penalty and argmax; max
relative error <= 1e-2 against the oracle's fp32 mode for float work.

The reference's semantics this pins at the boundary: launch_fused_attn_block
and launch_fused_mlp_stage1 take an already-normalised x and ignore
norm_weight / eps (src/kernels.cu:502, :576); launch_rmsnorm takes eps as
half (src/kernels.cu:689-768)."""
import json
import os
import subprocess

import numpy as np
import pytest

import cuqwen_amd as cq
from oracle import oracle as orc
from tests.gpu_util import rel_err

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOL = 1e-2
QUANT = {"fp16": 0, "int8": 1, "int4": 2}
MODEL = {"0_5b": "0.5B", "1_5b": "1.5B"}


def _caller(model, quant):
    return os.path.join(ROOT, "tests", "compat", f"kernel_caller_{model}_{quant}")


def _run(exe, *args):
    print(os.path.basename(exe), *args, flush=True)
    r = subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


class Dump:
    def __init__(self, d):
        self.d = d

    def __call__(self, name, dtype, shape=None):
        a = np.fromfile(os.path.join(self.d, name + ".bin"), dtype=dtype)
        return a.reshape(shape) if shape is not None else a


@pytest.mark.parametrize("model,quant,pos", [("0_5b", "int8", 16000), ("0_5b", "int4", 777), ("0_5b", "fp16", 0),
                                             ("1_5b", "int4", 16000)])
def test_kernel_profile_sequence(tmp_path, model, quant, pos):
    out = _run(_caller(model, quant), "ops", tmp_path, pos)
    cfg = cq.preset(MODEL[model], quant)
    q = QUANT[quant]
    d, I, V = cfg.dim, cfg.intermediate_size, cfg.vocab_size
    H, KV, hd = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    qd, kvd = H * hd, KV * hd
    f = Dump(str(tmp_path))
    h = np.float16

    def W(name, rows, cols):
        if q == 0:
            return f(name, h, (rows, cols)), None
        stride = cols if q == 1 else cols // 2
        return f(name, np.uint8, (rows, stride)), f("S" + name[1:], h, (rows, cols // 128))

    def gemv(name, rows, cols, x, mode=1):
        Wm, Sm = W(name, rows, cols)
        return orc.gemv(q, Wm, Sm, x, rows, cols, 128, mode=mode)

    x0, nw = f("x0", h), f("norm_w", h)
    # 1. launch_rmsnorm (half eps)
    att = f("01_att", h)
    assert rel_err(att, orc.rmsnorm(x0, nw, mode=1)) <= TOL
    # 2. launch_fused_attn_block on the normalised att: half(W att + b), RoPE at pos
    proj = {n: (gemv("W" + n, r, d, att) + f("b" + n, h).astype(np.float32)).astype(h)
            for n, r in (("q", qd), ("k", kvd), ("v", kvd))}
    gq, gk, gv = f("02_q", h), f("02_k", h), f("02_v", h)
    assert rel_err(gq, orc.rope(proj["q"], H, hd, pos)) <= TOL
    assert rel_err(gk, orc.rope(proj["k"], KV, hd, pos)) <= TOL
    assert rel_err(gv, proj["v"]) <= TOL
    # 3. launch_kv_cache_store: row pos of each head, neighbours untouched
    lo, hi = max(pos - 1, 0), min(pos + 1, cfg.max_seq_len - 1)
    rows = f("03_kv_rows", h, (2, KV, hi - lo + 1, hd))
    kpre, vpre = f("kc_prefix", h, (KV, pos, hd)), f("vc_prefix", h, (KV, pos, hd))
    for c, (new, pre) in enumerate(((gk, kpre), (gv, vpre))):
        assert np.array_equal(rows[c, :, pos - lo].view(np.uint16), new.reshape(KV, hd).view(np.uint16))
        if pos > 0:
            assert np.array_equal(rows[c, :, 0].view(np.uint16), pre[:, pos - 1].view(np.uint16))
        if hi > pos:
            assert not rows[c, :, hi - lo].any()
    # 4. launch_gqa_attention_decode over keys [0, pos]
    K = np.concatenate([kpre, gk.reshape(KV, 1, hd)], axis=1)
    Vc = np.concatenate([vpre, gv.reshape(KV, 1, hd)], axis=1)
    xb = f("04_xb", h)
    assert rel_err(xb, orc.attention(gq, K, Vc, H, KV, hd, pos + 1, mode=1)) <= TOL
    # 5. launch_gemv_add_fp16: x = half(x + Wo xb)
    x5 = f("05_x", h)
    assert rel_err(x5, x0.astype(np.float32) + gemv("Wo", d, qd, xb)) <= TOL
    # 6. launch_fused_mlp_stage1 on att (no norm): silu(g) * u
    gg = gemv("Wg", I, d, att).astype(np.float64)
    uu = gemv("Wu", I, d, att).astype(np.float64)
    gate = f("06_gate", h)
    assert rel_err(gate, gg / (1 + np.exp(-gg)) * uu) <= TOL
    # 7. launch_fused_mlp_stage2: x = half(x + Wd gate)
    x7 = f("07_x", h)
    assert rel_err(x7, x5.astype(np.float32) + gemv("Wd", d, I, gate)) <= TOL
    # 8. launch_embedding_lookup
    x8 = f("08_x", h)
    assert np.array_equal(x8.view(np.uint16), f("embed_row", h).view(np.uint16))
    # 9. final launch_rmsnorm
    xb9 = f("09_xb", h)
    assert rel_err(xb9, orc.rmsnorm(x8, nw, mode=1)) <= TOL
    # 10. launch_compute_logits (fp16 head)
    l10 = f("10_logits", h)
    assert rel_err(l10, orc.gemv(0, f("lmhead", h, (V, d)), None, xb9, V, d, mode=1)) <= TOL
    # 11. launch_apply_repetition_penalty: each distinct id once, bit-exact
    l11 = f("11_logits", h)
    assert np.array_equal(l11.view(np.uint16), orc.penalty(l10, f("hist", np.int32)).view(np.uint16))
    # 12. launch_argmax: bit-exact (ties -> lowest index)
    assert int(f("12_samp", np.int32)[0]) == orc.argmax(l11)
    # 13. launch_compute_logits_int8 and 14. a second launch_argmax
    l13 = f("13_logits", h)
    want13 = orc.gemv(1, f("lmq", np.uint8, (V, d)), f("lms", h, (V, d // 128)), xb9, V, d, mode=1)
    assert rel_err(l13, want13) <= TOL
    assert int(f("14_samp", np.int32)[0]) == orc.argmax(l13)
    assert out["pos"] == pos


@pytest.mark.parametrize("quant", ["int8", "int4", "fp16"])
def test_loaded_o_proj_weight_is_exporter_layout(tmp_path, quant):
    """LayerWeights.o_proj_weight / o_proj_scale from the compat load_weights
    are the exporter's row-major Wo (the engine keeps panels), so
    launch_gemv_add_fp16 on them, as src/model.cu:129 runs it, gives
    x + Wo xb with the file's Wo."""
    cfg = cq.preset("0.5B", quant)
    path = str(tmp_path / f"model_{quant}_0_5b.bin")
    cq.write_synthetic_file(path, cfg, 9)
    try:
        d, qd, q = cfg.dim, cfg.n_heads * cfg.head_dim, QUANT[quant]
        om = orc.Model.synth(cfg, 9, 16)   # the generator the file was written from (tested bit-identical)
        for layer in (0, cfg.n_layers - 1):
            _run(_caller("0_5b", quant), "oproj", path, tmp_path, layer)
            f = Dump(str(tmp_path))
            xb, x0, x1 = f("xb", np.float16), f("x0", np.float16), f("x1", np.float16)
            if q == 0:
                Wm, Sm = om.tensor(layer, orc.K_WO, 0).view(np.float16).reshape(d, qd), None
            else:
                Wm = om.tensor(layer, orc.K_WO, 0).reshape(d, -1)
                Sm = om.tensor(layer, orc.K_WO, 1).view(np.float16).reshape(d, qd // 128)
            assert rel_err(x1, x0.astype(np.float32) + orc.gemv(q, Wm, Sm, xb, d, qd, 128, mode=1)) <= TOL
    finally:
        os.remove(path)


def test_wo_rows_equal_file_bytes():
    """cq_weights_wo_rows returns the file's Wo bytes and scales exactly
    (the inverse of the engine's panel conversion), for every layer."""
    import ctypes
    from tests.conftest import tiny_config
    for quant in (0, 1, 2):
        cfg = tiny_config(quant, n_layers=3)
        w = cq.synth_weights(cfg, 4)
        om = orc.Model.synth(cfg, 4, 16)
        d, qd = cfg.dim, cfg.n_heads * cfg.head_dim
        for layer in range(cfg.n_layers):
            pw, ps = ctypes.c_void_p(), ctypes.c_void_p()
            cq.check(cq.lib.cq_weights_wo_rows(w.handle, layer, ctypes.byref(pw), ctypes.byref(ps)))
            want_w = om.tensor(layer, orc.K_WO, 0)
            got_w = np.zeros(want_w.size, np.uint8)
            cq.check(cq.lib.cq_memcpy_d2h(got_w.ctypes.data, pw.value, got_w.size))
            assert np.array_equal(got_w, want_w)
            if quant:
                want_s = om.tensor(layer, orc.K_WO, 1)
                got_s = np.zeros(want_s.size, np.uint8)
                cq.check(cq.lib.cq_memcpy_d2h(got_s.ctypes.data, ps.value, got_s.size))
                assert np.array_equal(got_s, want_s)
            else:
                assert ps.value is None
        assert d * qd > 0
        w.free()


@pytest.mark.parametrize("max_kernels", [3, 4, 16])
def test_profile_leaves_the_step_unchanged(max_kernels):
    """cq_state_profile runs the per-layer kernels on the state's buffers; a
    profile that stops after the merged O-projection (3) or gate/up (4) must
    not leave O-projection sums behind for the next step."""
    from tests.conftest import tiny_config
    cfg = tiny_config(2)
    w = cq.synth_weights(cfg, 8)
    a, b = cq.State(cfg, w), cq.State(cfg, w)
    try:
        ta = a.forward(5, 0)
        tb = b.forward(5, 0)
        # at a position the next step does not attend (the profile's QKV
        # launches write that cache row)
        b.profile(100, iters=1, max_kernels=max_kernels)
        ta2, tb2 = a.forward(ta, 1, [ta]), b.forward(tb, 1, [tb])
        assert ta2 == tb2
        np.testing.assert_array_equal(a.logits().view(np.uint16), b.logits().view(np.uint16))
    finally:
        a.free()
        b.free()
        w.free()
