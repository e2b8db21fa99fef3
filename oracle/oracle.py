"""ctypes binding of the CPU oracle (oracle/weaver_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, to check results (or as the timed CPU port), never by
the product package.  Functions take the host arrays produced by
``aether_nexus_amd.workloads.host_arrays`` plus the workload geometry.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

from aether_nexus_amd.types import AW_F_CAUSAL, DecodeDesc

HERE = Path(__file__).resolve().parent
# WEAVER_ORACLE_LIB: another build of the same source (the sanitizer run's).
LIB = Path(os.environ.get("WEAVER_ORACLE_LIB") or HERE / "libweaver_oracle.so")
SRC = HERE / "weaver_oracle.c"

_lib = None


def build() -> Path:
    """Compile the oracle with gcc (no fast-math; fp contraction off)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "libweaver_oracle.so"], check=True)
    return LIB


def build_native(out: Path) -> Path:
    """Compile the same source for the host that runs it (-O3 -march=native,
    fp contraction off) into `out`: the timed CPU baseline's build."""
    subprocess.run(["make", "-s", "-C", str(HERE), "native", f"NATIVE_OUT={out}"], check=True,
                   stdout=subprocess.DEVNULL)
    return out


def use_lib(path: Path) -> None:
    """Bind the oracle functions to another build of the same source."""
    global _lib
    _lib = _bind(ctypes.CDLL(str(path)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.is_file():
            build()
        _lib = _bind(ctypes.CDLL(str(LIB)))
    return _lib


def _bind(l: ctypes.CDLL) -> ctypes.CDLL:
    """Argument and result types of the exported functions."""
    vp, u64 = ctypes.c_void_p, ctypes.c_uint64
    l.or_h2f.restype = ctypes.c_float
    l.or_h2f.argtypes = [ctypes.c_uint16]
    l.or_f2h.restype = ctypes.c_uint16
    l.or_f2h.argtypes = [ctypes.c_float]
    l.or_h2f_array.argtypes = [vp, vp, ctypes.c_size_t]
    l.or_f2h_array.argtypes = [vp, vp, ctypes.c_size_t]
    l.or_decode_ref32.argtypes = [vp, ctypes.c_int]
    l.or_decode_ref32_rows.argtypes = [vp, vp, u64, vp, ctypes.c_int]
    l.or_decode_f64.argtypes = [vp, vp, u64, vp, ctypes.c_int]
    l.or_qlatent_f64.argtypes = [vp, vp]
    l.or_gather_codes.argtypes = [vp, u64, vp, ctypes.c_uint32, ctypes.c_uint32, vp, vp, vp]
    l.or_encode_blocks.argtypes = [vp, u64, ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_uint32, ctypes.c_uint32,
                                   vp, vp, ctypes.c_uint32, vp, u64, ctypes.c_int, vp]
    l.or_block_entropy.argtypes = [vp, u64]
    l.or_block_entropy.restype = ctypes.c_float
    for f in ("or_decode_ref32", "or_decode_ref32_rows", "or_decode_f64", "or_qlatent_f64", "or_gather_codes",
              "or_encode_blocks"):
        getattr(l, f).restype = ctypes.c_int
    return l


class OracleError(RuntimeError):
    pass


def _p(a):
    return None if a is None else a.ctypes.data


def host_desc(geom, arrs: dict, out: np.ndarray | None = None) -> tuple[DecodeDesc, list]:
    """aw_decode_desc over host numpy arrays (kept alive by the returned list)."""
    keep = []

    def c(a, dt):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=dt)
        keep.append(a)
        return a

    d = DecodeDesc()
    d.layers, d.batch, d.queries = geom.layers, geom.batch, geom.queries
    d.q_heads, d.kv_heads, d.head_dim = geom.q_heads, geom.kv_heads, geom.head_dim
    d.dict_size, d.dict_heads = geom.dict_size, geom.dict_heads
    d.hot_count, d.cold_count = geom.hot_count, geom.cold_count
    d.refs_stride = max(geom.refs_stride, 1)
    d.flags = AW_F_CAUSAL if geom.causal else 0
    d.scale = geom.scale
    d.hot_blocks, d.cold_blocks = geom.hot_blocks, geom.cold_blocks
    d.q = _p(c(arrs["q"], np.uint16))
    d.q_latent = _p(c(arrs.get("q_latent"), np.uint16))
    d.hot_k = _p(c(arrs.get("hot_k"), np.uint16))
    d.hot_v = _p(c(arrs.get("hot_v"), np.uint16))
    d.cold = _p(c(arrs.get("cold"), np.uint16))
    d.refs = _p(c(arrs["refs"], np.uint32))
    d.seq_hot = _p(c(arrs.get("seq_hot"), np.uint32))
    d.seq_cold = _p(c(arrs.get("seq_cold"), np.uint32))
    d.dict = _p(c(arrs.get("dictionary"), np.uint16))
    if out is not None:
        keep.append(out)
        d.out = out.ctypes.data
    return d, keep


def n_rows(geom) -> int:
    return geom.layers * geom.batch * geom.queries * geom.q_heads


def decode_ref32(geom, arrs: dict, threads: int = 8) -> np.ndarray:
    """fp32 restatement of weaver_kernel.metal -> f16 [L,B,Q,Hq,d] (as float16)."""
    out = np.zeros(n_rows(geom) * geom.head_dim, dtype=np.uint16)
    d, keep = host_desc(geom, arrs, out)
    rc = lib().or_decode_ref32(ctypes.byref(d), threads)
    if rc:
        raise OracleError(f"or_decode_ref32 failed: {rc}")
    return out.view(np.float16).reshape(geom.layers, geom.batch, geom.queries, geom.q_heads, geom.head_dim)


def decode_ref32_rows(geom, arrs: dict, rows, threads: int = 8) -> np.ndarray:
    rows = np.ascontiguousarray(rows, dtype=np.uint64)
    out = np.zeros(rows.size * geom.head_dim, dtype=np.uint16)
    d, keep = host_desc(geom, arrs)
    rc = lib().or_decode_ref32_rows(ctypes.byref(d), rows.ctypes.data, rows.size, out.ctypes.data, threads)
    if rc:
        raise OracleError(f"or_decode_ref32_rows failed: {rc}")
    return out.view(np.float16).reshape(rows.size, geom.head_dim)


def decode_f64(geom, arrs: dict, rows=None, threads: int = 8) -> np.ndarray:
    """fp64 dense brute force.  rows=None: all rows -> [L,B,Q,Hq,d]; else [n, d]
    for row ids ((l*B + b)*Q + q)*Hq + h."""
    d, keep = host_desc(geom, arrs)
    if rows is None:
        out = np.zeros(n_rows(geom) * geom.head_dim, dtype=np.float64)
        rc = lib().or_decode_f64(ctypes.byref(d), None, 0, out.ctypes.data, threads)
        shape = (geom.layers, geom.batch, geom.queries, geom.q_heads, geom.head_dim)
    else:
        rows = np.ascontiguousarray(rows, dtype=np.uint64)
        out = np.zeros(rows.size * geom.head_dim, dtype=np.float64)
        rc = lib().or_decode_f64(ctypes.byref(d), rows.ctypes.data, rows.size, out.ctypes.data, threads)
        shape = (rows.size, geom.head_dim)
    if rc:
        raise OracleError(f"or_decode_f64 failed: {rc}")
    return out.reshape(shape)


def qlatent_f64(geom, arrs: dict) -> np.ndarray:
    out = np.zeros(n_rows(geom) * geom.dict_size, dtype=np.float64)
    d, keep = host_desc(geom, arrs)
    rc = lib().or_qlatent_f64(ctypes.byref(d), out.ctypes.data)
    if rc:
        raise OracleError(f"or_qlatent_f64 failed: {rc}")
    return out.reshape(geom.layers, geom.batch, geom.queries, geom.q_heads, geom.dict_size)


def gather_codes(codes_words: np.ndarray, dictionary_bits: np.ndarray, dict_size: int, head_dim: int):
    """(idx u32 [n*4], coef f32 [n*4], atoms u16 [n*4, head_dim]) — bit-exact decode."""
    w = np.ascontiguousarray(codes_words, dtype=np.uint16).reshape(-1, 8)
    dic = np.ascontiguousarray(dictionary_bits, dtype=np.uint16)
    n = w.shape[0]
    idx = np.zeros(n * 4, dtype=np.uint32)
    coef = np.zeros(n * 4, dtype=np.float32)
    atoms = np.zeros((n * 4, head_dim), dtype=np.uint16)
    rc = lib().or_gather_codes(w.ctypes.data, n, dic.ctypes.data, dict_size, head_dim, idx.ctypes.data,
                               coef.ctypes.data, atoms.ctypes.data)
    if rc:
        raise OracleError(f"or_gather_codes failed: {rc}")
    return idx, coef, atoms


def h2f(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.zeros(b.shape, dtype=np.float32)
    lib().or_h2f_array(b.ctypes.data, out.ctypes.data, b.size)
    return out


def f2h(vals: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(vals, dtype=np.float32)
    out = np.zeros(v.shape, dtype=np.uint16)
    lib().or_f2h_array(v.ctypes.data, out.ctypes.data, v.size)
    return out


def encode_blocks(hot: np.ndarray, dictionary: np.ndarray, src, dst=None, cold: np.ndarray | None = None,
                  head_blocked: bool = False, entropy: bool = False):
    """SparseCode encoder (distiller.rs:171-246) over host arrays.

    hot: f16 bits [hot_blocks, 16, kv_heads, head_dim] (uint16); dictionary: f16
    bits [dict_heads, dict_size, head_dim]; src / dst: block indices.  Returns the
    cold pool (uint16 words [cold_blocks, 16, kv_heads, 8], or [.., kv_heads, 16, 8]
    when head_blocked) with the encoded blocks written, and the blocks' entropy
    proxies when asked."""
    hot = np.ascontiguousarray(hot, dtype=np.uint16)
    dictionary = np.ascontiguousarray(dictionary, dtype=np.uint16)
    hb, bs, hkv, hd = hot.shape
    dh, a, hd2 = dictionary.shape
    assert bs == 16 and hd2 == hd
    src = np.ascontiguousarray(src, dtype=np.uint32)
    dsta = None if dst is None else np.ascontiguousarray(dst, dtype=np.uint32)
    if cold is None:
        nb = int(max(src.max(initial=0), 0 if dsta is None else dsta.max(initial=0))) + 1
        cold = np.zeros((nb, hkv, 16, 8) if head_blocked else (nb, 16, hkv, 8), dtype=np.uint16)
    cold = np.ascontiguousarray(cold, dtype=np.uint16)
    ent = np.zeros(src.size, dtype=np.float32) if entropy else None
    rc = lib().or_encode_blocks(hot.ctypes.data, hb, hkv, hd, dictionary.ctypes.data, a, dh, src.ctypes.data,
                                None if dsta is None else dsta.ctypes.data, src.size, cold.ctypes.data,
                                cold.shape[0], int(head_blocked), None if ent is None else ent.ctypes.data)
    if rc:
        raise OracleError(f"or_encode_blocks failed: {rc}")
    return (cold, ent) if entropy else cold


def block_entropy(vals: np.ndarray) -> float:
    """Variance proxy of one block's f16 values (distiller.rs:126-159)."""
    v = np.ascontiguousarray(vals, dtype=np.uint16).ravel()
    return float(lib().or_block_entropy(v.ctypes.data, v.size))
