"""Writes tests/golden/quant_golden.npz: adversarial inputs for the
weight quantizer and the outputs of the exporter's numpy statements
(export_weights.py:123-146 int8, :161-183 int4, :197-199 packing), run here
with numpy exactly as the exporter runs them.

Cases: exact .5 ties after the fp32 division (round half to even), fp16
subnormal scales, an all-zero group, clipping, and random N(0, 0.02) rows.
Run: python tests/golden/make_quant_golden.py
"""
import os

import numpy as np

G = 128


def quant(arr, qmax):
    arr = arr.astype(np.float32)
    o, i = arr.shape
    grouped = arr.reshape(o, i // G, G)
    max_abs = np.max(np.abs(grouped), axis=2)
    scales = max_abs / float(qmax)
    safe = np.where(scales > 0.0, scales, 1.0)
    q = np.round(grouped / safe[:, :, None])
    q = np.clip(q, -qmax, qmax).astype(np.int8)
    return q.reshape(o, i), scales.astype(np.float16)


def pack4(q):
    o, i = q.shape
    nib = (q.astype(np.int16) & 0xF).astype(np.uint8).reshape(o, i // 2, 2)
    return (nib[:, :, 0] | (nib[:, :, 1] << 4)).astype(np.uint8)


def main():
    rng = np.random.default_rng(20240601)
    rows = []
    # ties for int8: max 127 -> scale 1.0; halves k + 0.5
    r = np.zeros(2 * G, dtype=np.float32)
    r[0] = 127.0
    r[1:G] = (np.arange(1, G) % 120) - 60 + 0.5
    r[G] = 127.0
    r[G + 1:] = -((np.arange(1, G) % 120) - 60 + 0.5)
    rows.append(r)
    # ties for int4: max 7 -> scale 1.0
    r = np.zeros(2 * G, dtype=np.float32)
    r[0] = 7.0
    r[1:G] = ((np.arange(1, G) % 14) - 7) + 0.5
    r[G] = -7.0
    r[G + 1:] = ((np.arange(1, G) % 8) - 4) + 0.5
    rows.append(r)
    # subnormal fp16 scales
    rows.append((rng.standard_normal(2 * G) * 3e-6).astype(np.float32))
    rows.append((rng.standard_normal(2 * G) * 2e-7).astype(np.float32))
    # zero group + tiny group
    r = np.zeros(2 * G, dtype=np.float32)
    r[G:] = rng.standard_normal(G) * 1e-3
    rows.append(r)
    # large values / wide range
    rows.append((rng.standard_normal(2 * G) * 300).astype(np.float32))
    for _ in range(26):
        rows.append((rng.standard_normal(2 * G) * 0.02).astype(np.float32))
    w = np.stack(rows).astype(np.float16)
    q8, s8 = quant(w, 127)
    q4, s4 = quant(w, 7)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_golden.npz")
    np.savez(out, w=w, int8_q=q8.view(np.uint8), int8_s=s8, int4_q=pack4(q4), int4_s=s4)
    print("wrote", out, w.shape)


if __name__ == "__main__":
    main()
