"""Writer of small weight files in the exporter's binary layout, for tests that
build models with hand-chosen tensors (export_weights.py:267-323: 256-byte
header of eleven int32, then embed, per-layer tensors, final norm, lm_head;
each quantized matrix is its weight block followed by its fp16 scale block).

Test infrastructure only.  Quantized matrices go through the oracle's
quantizer, which tests/test_oracle.py pins against the exporter's golden
vectors.
"""
import struct

import numpy as np

MAGIC = 0x5157454E


def write(path, cfg, t):
    """cfg: dict with vocab, dim, inter, layers, heads, kv, hd, max_seq, quant,
    lm_fmt (0 fp16-or-tied, 1 int8).  t: dict of fp16 arrays: embed[V,d],
    final_norm[d], lm_head[V,d] or None (tied), layers[l] = dict(in_norm, wq,
    bq, wk, bk, wv, bv, wo, post_norm, wg, wu, wd)."""
    from oracle import oracle as orc

    q = cfg["quant"]

    def mat(f, w, quant):
        w = np.ascontiguousarray(w, dtype=np.float16)
        if quant == 0:
            f.write(w.tobytes())
            return
        qq, s = orc.quantize(quant, w, 128)
        f.write(qq.tobytes())
        f.write(s.tobytes())

    def vec(f, v):
        f.write(np.ascontiguousarray(v, dtype=np.float16).tobytes())

    with open(path, "wb") as f:
        hdr = struct.pack("<11i", MAGIC, cfg["vocab"], cfg["dim"], cfg["inter"], cfg["layers"], cfg["heads"],
                          cfg["kv"], cfg["hd"], cfg["max_seq"], q, cfg["lm_fmt"])
        f.write(hdr + b"\0" * (256 - len(hdr)))
        vec(f, t["embed"])
        for L in t["layers"]:
            vec(f, L["in_norm"])
            mat(f, L["wq"], q)
            vec(f, L["bq"])
            mat(f, L["wk"], q)
            vec(f, L["bk"])
            mat(f, L["wv"], q)
            vec(f, L["bv"])
            mat(f, L["wo"], q)
            vec(f, L["post_norm"])
            mat(f, L["wg"], q)
            mat(f, L["wu"], q)
            mat(f, L["wd"], q)
        vec(f, t["final_norm"])
        if cfg["lm_fmt"] == 1:
            mat(f, t["lm_head"], 1)
        elif t.get("lm_head") is not None:
            mat(f, t["lm_head"], 0)


def zeros_model(cfg, rng):
    """Every projection weight and bias zero; embeddings and norm weights random."""
    d, I = cfg["dim"], cfg["inter"]
    qd, kvd = cfg["heads"] * cfg["hd"], cfg["kv"] * cfg["hd"]
    h = np.float16

    def norm():
        return (1.0 + 0.3 * rng.standard_normal(d)).astype(h)

    layers = []
    for _ in range(cfg["layers"]):
        layers.append(dict(in_norm=norm(), wq=np.zeros((qd, d), h), bq=np.zeros(qd, h), wk=np.zeros((kvd, d), h),
                           bk=np.zeros(kvd, h), wv=np.zeros((kvd, d), h), bv=np.zeros(kvd, h),
                           wo=np.zeros((d, qd), h), post_norm=norm(), wg=np.zeros((I, d), h),
                           wu=np.zeros((I, d), h), wd=np.zeros((d, I), h)))
    return dict(embed=(rng.standard_normal((cfg["vocab"], d)) * 0.5).astype(h), final_norm=norm(),
                lm_head=None, layers=layers)
