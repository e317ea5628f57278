"""ctypes loader for oracle/libgqa_oracle.so -- test infrastructure only.

Used by tests/ and by bench.py's cpu_baseline leg. Build with
``make -C oracle`` (``__graft_entry__.build()`` does it).
"""

import ctypes
import os

import numpy as np

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgqa_oracle.so")
_lib = None

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise FileNotFoundError(f"{_LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_attention_ref.argtypes = [_u16p, _u16p, _u16p, _i32p, _i32p, _f32p,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                           ctypes.c_int]
        L.oracle_attention_ref.restype = ctypes.c_int
        L.oracle_kv_offset.argtypes = [_i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int]
        L.oracle_kv_offset.restype = ctypes.c_int64
        L.oracle_partial_state.argtypes = [_u16p, _u16p, _u16p, _i32p, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_float,
                                           ctypes.POINTER(ctypes.c_double),
                                           ctypes.POINTER(ctypes.c_double), _f64p]
        L.oracle_partial_state.restype = None
        L.oracle_merge_states.argtypes = [ctypes.c_int, _f64p, _f64p, _f64p, ctypes.c_int, _f64p]
        L.oracle_merge_states.restype = None
        L.oracle_mla_decode.argtypes = [_u16p, _u16p, _i32p, _i32p, _f32p, _f32p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.oracle_mla_decode.restype = ctypes.c_int
        _lib = L
    return _lib


def attention_ref(q, k_cache, v_cache, block_table, seq_lens, scale, nthreads=0):
    """fp32 [B, Hq, 128]; bf16 inputs as uint16 arrays of raw bits."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k_cache = np.ascontiguousarray(k_cache, dtype=np.uint16)
    v_cache = np.ascontiguousarray(v_cache, dtype=np.uint16)
    block_table = np.ascontiguousarray(block_table, dtype=np.int32)
    seq_lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    B, Hq, _ = q.shape
    _, bs, Hkv, _ = k_cache.shape
    out = np.empty((B, Hq, 128), dtype=np.float32)
    rc = lib().oracle_attention_ref(q, k_cache, v_cache, block_table, seq_lens, out, B, Hq, Hkv,
                                    bs, block_table.shape[1], float(scale), int(nthreads))
    if rc != 0:
        raise ValueError("oracle_attention_ref rejected its arguments")
    return out


def kv_offset(bt_row, t, block_size, Hkv, hkv):
    return lib().oracle_kv_offset(np.ascontiguousarray(bt_row, dtype=np.int32), t, block_size,
                                  Hkv, hkv)


def partial_state(q_vec, k_cache, v_cache, bt_row, hkv, start, end, scale):
    """(m, l, acc[128]) over tokens [start, end) of one request."""
    _, bs, Hkv, _ = k_cache.shape
    m = ctypes.c_double()
    l = ctypes.c_double()
    acc = np.zeros(128, dtype=np.float64)
    lib().oracle_partial_state(np.ascontiguousarray(q_vec, dtype=np.uint16),
                               np.ascontiguousarray(k_cache, dtype=np.uint16),
                               np.ascontiguousarray(v_cache, dtype=np.uint16),
                               np.ascontiguousarray(bt_row, dtype=np.int32), bs, Hkv, hkv, start,
                               end, float(scale), ctypes.byref(m), ctypes.byref(l), acc)
    return m.value, l.value, acc


def merge_states(ms, ls, accs):
    ms = np.ascontiguousarray(ms, dtype=np.float64)
    ls = np.ascontiguousarray(ls, dtype=np.float64)
    accs = np.ascontiguousarray(accs, dtype=np.float64)
    out = np.empty(accs.shape[1], dtype=np.float64)
    lib().oracle_merge_states(len(ms), ms, ls, accs, accs.shape[1], out)
    return out


def mla_decode_ref(q, kv_cache, block_table, seq_lens, scale, causal=False, dv=512, nthreads=0):
    """MLA decode in double precision (oracle/mla_decode_oracle.c):
    (out [B, s_q, h_q, dv] float32, lse [B, h_q, s_q] float32); bf16 inputs
    as uint16 arrays of raw bits."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    kv_cache = np.ascontiguousarray(kv_cache, dtype=np.uint16)
    block_table = np.ascontiguousarray(block_table, dtype=np.int32)
    seq_lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    B, s_q, h_q, _ = q.shape
    bs = kv_cache.shape[1]
    out = np.empty((B, s_q, h_q, dv), dtype=np.float32)
    lse = np.empty((B, h_q, s_q), dtype=np.float32)
    rc = lib().oracle_mla_decode(q, kv_cache, block_table, seq_lens, out, lse, B, s_q, h_q, bs,
                                 block_table.shape[1], dv, float(scale), int(bool(causal)),
                                 int(nthreads))
    if rc != 0:
        raise ValueError("oracle_mla_decode rejected its arguments or ran out of memory")
    return out, lse
