"""ctypes binding of the CPU export oracle (oracle/export.cpp) and a parser of
the quantised .bin layouts it writes.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product never uses it.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np

from .ffi import lib

ARCH_NAMES = ("HalfKP", "HalfKaSplit", "HalfKaMerged", "HalfKaHmSplit", "HalfKaHmMerged")
ACTIVATIONS = {"crelu": 0, "screlu": 1, "pairwise": 2}
# orc_quantise kinds
Q_LS_I16, Q_LS_I8, Q_LS_I32, Q_SIMPLE_I16, Q_SIMPLE_I8, Q_SIMPLE_I32 = range(6)


def _P(a):
    return a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _sig():
    L = lib()
    L.orc_leb128_encode.restype = C.c_int64
    L.orc_leb128_decode_one.restype = C.c_int32
    L.orc_leb128_decode_i16.restype = C.c_int64
    L.orc_pad32.restype = C.c_uint64
    L.orc_pad32.argtypes = [C.c_uint64]
    for name in ("orc_ls_fc_hash", "orc_ls_network_hash", "orc_simple_fc_hash", "orc_simple_network_hash"):
        getattr(L, name).restype = C.c_uint32
    L.orc_ls_fc_hash.argtypes = [C.c_uint64, C.c_uint64]
    L.orc_ls_network_hash.argtypes = [C.c_uint32, C.c_uint64, C.c_uint64]
    L.orc_simple_fc_hash.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
    L.orc_simple_network_hash.argtypes = [C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_int32]
    L.orc_ls_arch_str.restype = C.c_int64
    L.orc_ls_arch_str.argtypes = [C.c_char_p] + [C.c_uint64] * 5 + [C.c_int32, C.c_int32, C.c_char_p, C.c_int64]
    L.orc_simple_arch_str.restype = C.c_int64
    L.orc_simple_arch_str.argtypes = [C.c_char_p] + [C.c_uint64] * 4 + [C.c_int32, C.c_int32, C.c_char_p,
                                                                         C.c_int64]
    L.orc_simple_fv_scale.restype = C.c_int32
    L.orc_simple_fv_scale.argtypes = [C.c_float]
    L.orc_ls_export_fv_scale.restype = C.c_int32
    L.orc_ls_export_fv_scale.argtypes = [C.c_int32, C.c_int32, C.c_int32, C.c_float, C.POINTER(C.c_int32)]
    L.orc_ls_save_quantised.restype = C.c_int64
    L.orc_ls_save_quantised.argtypes = ([C.c_char_p, C.c_uint32] + [C.c_uint64] * 5 + [C.c_void_p] * 10 +
                                        [C.c_int32, C.c_int32, C.c_void_p, C.c_int64])
    L.orc_simple_save_quantised.restype = C.c_int64
    L.orc_simple_save_quantised.argtypes = ([C.c_char_p, C.c_uint32] + [C.c_uint64] * 4 +
                                            [C.c_int32, C.c_int32] + [C.c_void_p] * 8 + [C.c_void_p, C.c_int64])
    return L


_L = None


def L():
    global _L
    if _L is None:
        _L = _sig()
    return _L


def leb128_encode(values) -> bytes:
    v = np.ascontiguousarray(values, dtype=np.int64)
    out = np.zeros(max(1, 10 * v.size), np.uint8)
    n = L().orc_leb128_encode(_P(v), C.c_int64(v.size), _P(out))
    return out[:n].tobytes()


def leb128_decode_one(data: bytes):
    buf = np.frombuffer(bytes(data) or b"\0", np.uint8).copy()
    val, used = C.c_int64(), C.c_int64()
    rc = L().orc_leb128_decode_one(_P(buf), C.c_int64(len(data)), C.byref(val), C.byref(used))
    if rc:
        raise ValueError({-1: "unexpected end of LEB128 data", -2: "LEB128 overflow"}[rc])
    return val.value, used.value


def leb128_decode_i16(data: bytes) -> np.ndarray:
    buf = np.frombuffer(bytes(data), np.uint8).copy()
    out = np.zeros(len(data), np.int16)
    n = L().orc_leb128_decode_i16(_P(buf), C.c_int64(len(data)), out.ctypes.data_as(C.c_void_p),
                                  C.c_int64(out.size))
    if n < 0:
        raise ValueError("bad LEB128 stream")
    return out[:n].copy()


def quantise(values, scale: float, kind: int) -> np.ndarray:
    v = _f32(values).ravel()
    out = np.zeros(v.size, np.int64)
    L().orc_quantise(_P(v), C.c_int64(v.size), C.c_double(scale), C.c_int32(kind), _P(out))
    return out


def pad32(x: int) -> int:
    return int(L().orc_pad32(x))


def ls_fc_hash(ft_out, l2_out) -> int:
    return int(L().orc_ls_fc_hash(ft_out, l2_out))


def ls_network_hash(feature_hash, ft_out, l2_out) -> int:
    return int(L().orc_ls_network_hash(feature_hash, ft_out, l2_out))


def simple_fc_hash(l1_input, l1_out, l2_out) -> int:
    return int(L().orc_simple_fc_hash(l1_input, l1_out, l2_out))


def simple_network_hash(feature_hash, ft_out, l1_out, l2_out, activation="crelu") -> int:
    return int(L().orc_simple_network_hash(feature_hash, ft_out, l1_out, l2_out, ACTIVATIONS[activation]))


def ls_arch_str(name, input_size, ft_out, l1_out, l2_in, l2_out, fv_scale=None) -> str:
    buf = C.create_string_buffer(4096)
    n = L().orc_ls_arch_str(name.encode(), input_size, ft_out, l1_out, l2_in, l2_out,
                            int(fv_scale is not None), int(fv_scale or 0), buf, 4096)
    return buf.raw[:n].decode()


def simple_arch_str(name, ft_in, ft_out, l1_out, l2_out, fv_scale, activation="crelu") -> str:
    buf = C.create_string_buffer(4096)
    n = L().orc_simple_arch_str(name.encode(), ft_in, ft_out, l1_out, l2_out, ACTIVATIONS[activation],
                                fv_scale, buf, 4096)
    return buf.raw[:n].decode()


def simple_fv_scale(scale: float) -> int:
    return int(L().orc_simple_fv_scale(scale))


def ls_export_fv_scale(override, loss_kind: int, score_scale: float):
    v = C.c_int32()
    has = L().orc_ls_export_fv_scale(int(override is not None), int(override or 0), loss_kind, score_scale,
                                     C.byref(v))
    return v.value if has else None


def coalesce(w_train, ft_in, piece_inputs, ft_out) -> np.ndarray:
    w = _f32(w_train)
    out = np.zeros(ft_in * ft_out, np.float32)
    L().orc_coalesce(_P(w), C.c_int64(ft_in), C.c_int64(piece_inputs), C.c_int64(ft_out), _P(out))
    return out


def ls_save_quantised(feature_set: int, feature_hash: int, ft_in, ft_out, l1_out, l2_out, nb, w: dict,
                      fv_scale=None) -> bytes:
    """LayerStackWeights::save_quantised; w holds export-shape f32 tensors by reference name."""
    names = ("ft_w", "ft_b", "l1_w", "l1_b", "l1_shared_weight", "l1_shared_bias", "l2_w", "l2_b", "l3_w", "l3_b")
    arrs = [_f32(w[k]).ravel() for k in names]
    cap = 3 * (ft_in * ft_out + ft_out) + (1 << 16) + nb * (l1_out * (ft_out + 64) + 4096)
    out = np.zeros(cap, np.uint8)
    n = L().orc_ls_save_quantised(ARCH_NAMES[feature_set].encode(), feature_hash, ft_in, ft_out, l1_out, l2_out,
                                  nb, *[_P(a) for a in arrs], int(fv_scale is not None), int(fv_scale or 0),
                                  _P(out), cap)
    assert n <= cap
    return out[:n].tobytes()


def simple_save_quantised(feature_set: int, feature_hash: int, ft_in, ft_out, l1_out, l2_out, w: dict,
                          fv_scale: int, activation="crelu") -> bytes:
    """SimpleWeights::save_quantised; l1_w (l1_out, l1_in) and l2_w (l2_out, l1_out) out-major."""
    names = ("ft_w", "ft_b", "l1_w", "l1_b", "l2_w", "l2_b", "l3_w", "l3_b")
    arrs = [_f32(w[k]).ravel() for k in names]
    cap = 2 * (ft_in * ft_out + ft_out) + (1 << 16) + l1_out * (2 * ft_out + 64) + 4096
    out = np.zeros(cap, np.uint8)
    n = L().orc_simple_save_quantised(ARCH_NAMES[feature_set].encode(), feature_hash, ft_in, ft_out, l1_out,
                                      l2_out, ACTIVATIONS[activation], fv_scale, *[_P(a) for a in arrs],
                                      _P(out), cap)
    assert n <= cap
    return out[:n].tobytes()


class _Reader:
    def __init__(self, buf: bytes):
        self.b, self.p = buf, 0

    def take(self, n):
        if self.p + n > len(self.b):
            raise ValueError("truncated file")
        s = self.b[self.p:self.p + n]
        self.p += n
        return s

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def i32s(self, n):
        return np.frombuffer(self.take(4 * n), "<i4").copy()

    def i8s(self, n):
        return np.frombuffer(self.take(n), np.int8).copy()

    def i16s(self, n):
        return np.frombuffer(self.take(2 * n), "<i2").copy()

    def leb(self):
        if self.take(17) != b"COMPRESSED_LEB128":
            raise ValueError("expected COMPRESSED_LEB128 magic")
        n = self.u32()
        return leb128_decode_i16(self.take(n)), n


def parse_layerstack(buf: bytes, ft_out: int, l1_out: int, l2_out: int) -> dict:
    """Splits a LayerStack .bin into its fields (layout of save_quantised, layerstack_weights.rs:568-829)."""
    r = _Reader(buf)
    d = dict(version=r.u32(), network_hash=r.u32())
    d["arch"] = r.take(r.u32()).decode()
    d["num_buckets"] = nb = r.u32()
    d["ft_hash"] = r.u32()
    d["ft_b"], _ = r.leb()
    d["ft_w"], d["ft_w_bytes"] = r.leb()
    l2_in = 2 * (l1_out - 1)
    stacks = []
    for _ in range(nb):
        s = dict(fc_hash=r.u32())
        s["l1_b"] = r.i32s(l1_out)
        s["l1_w"] = r.i8s(l1_out * pad32(ft_out)).reshape(l1_out, -1)
        s["l2_b"] = r.i32s(l2_out)
        s["l2_w"] = r.i8s(l2_out * pad32(l2_in)).reshape(l2_out, -1)
        s["l3_b"] = r.i32s(1)
        s["l3_w"] = r.i8s(pad32(l2_out))
        stacks.append(s)
    d["stacks"] = stacks
    d["trailing"] = len(buf) - r.p
    return d


def parse_simple(buf: bytes, ft_in: int, ft_out: int, l1_out: int, l2_out: int, activation="crelu") -> dict:
    """Splits a Simple .bin into its fields (layout of SimpleWeights::save_quantised)."""
    l1_in = 2 * ft_out // (2 if activation == "pairwise" else 1)
    r = _Reader(buf)
    d = dict(version=r.u32(), network_hash=r.u32())
    d["arch"] = r.take(r.u32()).decode()
    d["ft_hash"] = r.u32()
    d["ft_b"] = r.i16s(ft_out)
    d["ft_w"] = r.i16s(ft_in * ft_out)
    d["fc_hash"] = r.u32()
    d["l1_b"] = r.i32s(l1_out)
    d["l1_w"] = r.i8s(l1_out * pad32(l1_in)).reshape(l1_out, -1)
    d["l2_b"] = r.i32s(l2_out)
    d["l2_w"] = r.i8s(l2_out * pad32(l1_out)).reshape(l2_out, -1)
    d["l3_b"] = r.i32s(1)
    d["l3_w"] = r.i8s(pad32(l2_out))
    d["trailing"] = len(buf) - r.p
    return d
