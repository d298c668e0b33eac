"""Helpers shared by the GPU tests."""
import numpy as np

import cuqwen_amd as cq

D = cq.DeviceBuffer


class Pool:
    """Owns every device buffer of one test until the test ends, so no
    pointer handed to a kernel can be released while the kernel may run."""

    def __init__(self):
        self.bufs = []

    def put(self, a):
        """Upload `a` (None -> NULL); returns the device pointer."""
        if a is None:
            return None
        b = D.from_array(np.ascontiguousarray(a))
        self.bufs.append(b)
        return b.ptr

    def i32(self, v):
        return self.put(np.array(v, dtype=np.int32).reshape(-1))

    def empty(self, nbytes, zero=False):
        b = D(nbytes)
        if zero:
            b.zero()
        self.bufs.append(b)
        return b

    def close(self):
        cq.synchronize()
        for b in self.bufs:
            b.free()
        self.bufs = []


def rel_err(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def k_offsets(n_kv, T, hd, max_seq):
    """Vectorised kv_k_offset (cq_common.h) for [n_kv][T][hd]."""
    h, t, d = np.meshgrid(np.arange(n_kv), np.arange(T), np.arange(hd), indexing="ij")
    kk, j, e = d >> 5, (d >> 3) & 3, d & 7
    return h * max_seq * hd + (t >> 4) * 16 * hd + ((kk * 64 + j * 16 + (t & 15)) * 8 + e)


def v_offsets(n_kv, T, hd, max_seq):
    h, t, d = np.meshgrid(np.arange(n_kv), np.arange(T), np.arange(hd), indexing="ij")
    dt, dl = d >> 4, d & 15
    t32 = t & 31
    j = (t32 & 15) >> 2
    e = (t32 & 3) + ((t32 >> 4) << 2)
    return h * max_seq * hd + (t >> 5) * 32 * hd + ((dt * 64 + j * 16 + dl) * 8 + e)


def k8_offsets(n_kv, T, hd, max_seq):
    """Vectorised kv8_k_offset (cq_common.h): byte offsets in an int8 / E4M3
    cache, operand pieces of instruction pairs side by side."""
    h, t, d = np.meshgrid(np.arange(n_kv), np.arange(T), np.arange(hd), indexing="ij")
    kk, j, e = d >> 5, (d >> 3) & 3, d & 7
    return h * max_seq * hd + (t >> 4) * 16 * hd + (((kk >> 1) * 64 + j * 16 + (t & 15)) * 16 + (kk & 1) * 8 + e)


def v8_offsets(n_kv, T, hd, max_seq):
    h, t, d = np.meshgrid(np.arange(n_kv), np.arange(T), np.arange(hd), indexing="ij")
    dt, dl = d >> 4, d & 15
    t32 = t & 31
    j = (t32 & 15) >> 2
    e = (t32 & 3) + ((t32 >> 4) << 2)
    return h * max_seq * hd + (t >> 5) * 32 * hd + (((dt >> 1) * 64 + j * 16 + dl) * 16 + (dt & 1) * 8 + e)


def tile_kv(K, V, max_seq):
    """Head-major K, V [n_kv][T][hd] -> the device cache layout."""
    n_kv, T, hd = K.shape
    kc = np.zeros(n_kv * max_seq * hd, dtype=np.float16)
    vc = np.zeros(n_kv * max_seq * hd, dtype=np.float16)
    kc[k_offsets(n_kv, T, hd, max_seq).ravel()] = K.ravel()
    vc[v_offsets(n_kv, T, hd, max_seq).ravel()] = V.ravel()
    return kc, vc
