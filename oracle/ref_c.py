"""Loader for the reference's own CPU kernel built by ``oracle/Makefile`` --
TEST INFRASTRUCTURE ONLY, see ``oracle/__init__``.

``vnni_source_gemm`` (``bench/vnni_source_kernel.c:8-47``) is the reference's
integer-exact A8 MXFP4 GEMM: qA = 512*A (e4m3 activations), qW = 2*W (E2M1
weights), per K32 block an exact integer dot computed as three unsigned byte
planes of qA + 2^18 against signed qW with ``dpbusd``, minus 2^18 * sum(qW),
then ``partial = dot * (1/1024) * sa * sw`` accumulated in fp32 in ascending
K32 order.  Its operand layout (``bench/vnni_source.py:48-84``): weights as
[N/8][K/4][8][4] int8 tiles, activations as three [M][K/4][8][4] byte planes
(each 4-byte K group repeated for the 8 output lanes), fp32 scales, int32
per-block weight sums.  This module prepares those operands from packed MXFP4
and e4m3 codes; it does not contain the reference code.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from . import codecs as C

REF_DIR = Path(__file__).resolve().parent / "_ref"


def _cpu_flags() -> set:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def library():
    """The build that this CPU can run, or None (not built / no VNNI)."""
    flags = _cpu_flags()
    cands = []
    if {"avx512_vnni", "avx512vl"} <= flags:
        cands.append("libvnni_source_avx512vnni.so")
    if "avx_vnni" in flags:
        cands.append("libvnni_source_avxvnni.so")
    for name in cands:
        p = REF_DIR / name
        if p.exists():
            lib = ctypes.CDLL(str(p))
            ptr = lambda dt: np.ctypeslib.ndpointer(dt, flags="C_CONTIGUOUS")
            lib.vnni_source_gemm.argtypes = [ptr(np.uint8), ptr(np.float32), ptr(np.int8), ptr(np.float32),
                                             ptr(np.int32), ptr(np.float32)] + [ctypes.c_int] * 3
            lib.vnni_source_gemm.restype = None
            return lib
    return None


def prepare_weights(packed: np.ndarray, scale: np.ndarray):
    """packed [N, K/2] + e8m0 [N, K/32] -> (tiled qW, fp32 sw, int32 block sums)."""
    n, kh = packed.shape
    k = 2 * kh
    if n % 8 or k % 128:
        raise ValueError("the reference kernel needs N % 8 == 0 and K % 128 == 0")
    qw = np.rint(C.decode_e2m1(packed).astype(np.float64) * 2).astype(np.int8)        # [N, K]
    tiled = np.ascontiguousarray(qw.reshape(n // 8, 8, k // 4, 4).transpose(0, 2, 1, 3))
    sums = qw.reshape(n, k // 32, 32).astype(np.int32).sum(-1).astype(np.int32)
    return tiled, C.e8m0_to_f32(scale).astype(np.float32), np.ascontiguousarray(sums)


def gemm(codes: np.ndarray, sa: np.ndarray, weights, lib=None) -> np.ndarray:
    """A8 GEMM of e4m3 codes [M, K] (+ scales [M, K/128]) against prepared weights -> fp32 [M, N]."""
    lib = lib or library()
    if lib is None:
        raise RuntimeError("reference C kernel not built or not runnable on this CPU")
    m, k = codes.shape
    qa = np.rint(C.e4m3_decode(codes).astype(np.float64) * 512).astype(np.int64)
    u = qa + 262144
    planes = np.stack([((u >> s) & 0xFF).astype(np.uint8) for s in (0, 8, 16)])     # [3, M, K]
    tiled_a = np.ascontiguousarray(np.broadcast_to(planes.reshape(3, m, k // 4, 1, 4), (3, m, k // 4, 8, 4)))
    tiled_w, sw, sums = weights
    n = sw.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    lib.vnni_source_gemm(tiled_a, np.ascontiguousarray(sa, dtype=np.float32), tiled_w, sw, sums, y, m, n, k)
    return y
