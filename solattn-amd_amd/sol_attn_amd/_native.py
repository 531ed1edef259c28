"""Launch layer over the HIP C-ABI library (replaces the reference's kernels.py).

Mirrors ``src/sol_attn_amd/kernels.py:185-225``: ``launch_sol`` and
``launch_dense`` take validated BF16 tensors, allocate every output and
workspace with ``torch.empty`` on the input device (the pooled key buffers
as one workspace), and enqueue the HIP kernels on the current stream.  There is no CPU path: when the library is not
built this module raises.
"""

from __future__ import annotations

import ctypes
import functools
import math
import os
import threading

import torch

BLOCK = 64
ABI_VERSION = 14

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsol_attn_amd.so")
_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i64p = ctypes.POINTER(ctypes.c_int64)
_dbl = ctypes.c_double
_int = ctypes.c_int

_SIGNATURES = {
    "sol_abi_version": ([], ctypes.c_int),
    "sol_last_error": ([], ctypes.c_char_p),
    "sol_pool_sizes": ([_i64, _i64, _i64, _i64, _i64p], ctypes.c_int),
    "sol_pool_kv": ([_p, _i64p, _p, _i64p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                     _p, _p, _p, _p, _p, _p], ctypes.c_int),
    "sol_pair_workspace_size": ([_i64, _i64, _i64, _i64], ctypes.c_int64),
    "sol_pair_strides": ([_p, _i64p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p], ctypes.c_int),
    "sol_split_workspace_size": ([_i64, _i64, _i64, _i64, _i64, _dbl, _i64], ctypes.c_int64),
    "sol_route_workspace_size": ([_i64, _i64, _i64, _i64, _dbl], ctypes.c_int64),
    "sol_attention_fwd": ([_p, _i64p, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64,
                           _p, _i64p, _p, _i64p,
                           _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                           _dbl, _dbl, _i64, _i64, _i64,
                           _p, _p, _p, _p, _p, _p, _p, _p, _int, _p], ctypes.c_int),
    "sol_dense_fwd": ([_p, _i64p, _p, _i64, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _i64,
                       _dbl, _p, _p, _p, _p], ctypes.c_int),
    "sol_plan_protection": ([_p, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _p, _p], ctypes.c_int),
    "sol_key_covariance_workspace_size": ([_i64, _i64, _i64], ctypes.c_int64),
    "sol_key_covariance": ([_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p], ctypes.c_int),
    "sol_quantize_keys": ([_p, _i64p, _p, _p, _i64, _i64, _i64, _i64, _i64, _int, _p, _p, _p], ctypes.c_int),
    "sol_attention_pools_keys": ([_i64, _i64, _i64, _i64, _i64], ctypes.c_int),
    "sol_attention_noalloc": ([_p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _i64,
                               _dbl, _dbl, _i64, _i64, _i64, _p, _p, _p], ctypes.c_int),
    "sol_attention_workspace_size": ([_i64, _i64, _i64, _i64, _i64, _dbl, _i64, _i64, _i64], ctypes.c_int64),
    "sol_attention_all_in": ([_p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _i64,
                              _dbl, _dbl, _i64, _i64, _i64, _p, _i64, _p, _p, _p], ctypes.c_int),
}


def library():
    """Load ``libsol_attn_amd.so`` once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"SOL HIP library not built ({LIB_PATH} missing); "
                "run `python -m sol_attn_amd._build` or __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.sol_abi_version() != ABI_VERSION:
            raise RuntimeError("libsol_attn_amd.so ABI version mismatch; rebuild it")
        _lib = lib
    return _lib


def _check(status):
    if status != 0:
        msg = library().sol_last_error().decode(errors="replace")
        raise RuntimeError(f"SOL HIP call failed ({status}): {msg}")


@functools.lru_cache(maxsize=512)
def _stride_array(batch, token, head):
    # Read-only once built: every call with the same strides shares one array.
    return (ctypes.c_int64 * 3)(batch, token, head)


def _strides(x, indexed=False):
    s = x.stride()
    return _stride_array(0 if indexed else s[0], s[-3], s[-2])


def _ptr(x):
    # ctypes passes a Python int (or None, NULL) for a c_void_p argument.
    return None if x is None else x.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device):
    """The device's current stream as a ``hipStream_t`` value."""
    if _raw_stream is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _aligned(x):
    """Rows start on 16-byte boundaries (base pointer and all strides)."""
    if x.data_ptr() & 15:
        return False
    for s in x.stride()[:-1]:
        if s & 7:
            return False
    return True


def _rows(x):
    # Misaligned views are copied once on the GPU; inputs are never written.
    return x if _aligned(x) else x.clone(memory_format=torch.contiguous_format)


def _tiles(b, h, nkb, d, device):
    return torch.empty((b, h, nkb, 2, BLOCK * d), device=device, dtype=torch.bfloat16)


def rows_mode(k, v, key_index=None, key_lengths=None):
    """Whether the attention kernels read key blocks straight from K / V rows
    (no pooled block tiles): plain strided keys of equal length, at least one
    block of them, token strides below 2^24 elements (``include/sol_attn_amd.h``)."""
    tk = k.shape[1]
    return (key_index is None and key_lengths is None and tk >= BLOCK
            and k.stride(1) < (1 << 24) and v.stride(1) < (1 << 24))


_ALIGN = 256  # byte alignment of each buffer carved from a workspace


@functools.lru_cache(maxsize=256)
def _carve(sizes):
    """Byte offsets of consecutive ``_ALIGN``-aligned regions (``sizes``: a tuple of
    byte counts), and their total."""
    offsets, total = [], 0
    for n in sizes:
        offsets.append(total)
        total += -(-n // _ALIGN) * _ALIGN
    return tuple(offsets), total


def _region(ws, offset, dtype, shape):
    n = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
    return ws[offset:offset + n].view(dtype).view(shape)


def pool_kv(k, v, key_index=None, moments=True, key_lengths=None, stream=None, views=True, qk_int8=False):
    """Centroid tiles, attention tiles and key moments (one HBM pass over K and V).

    ``k``/``v``: ``[B, Tk, H, D]`` BF16 or, with ``key_index`` ``[B, Tk]``,
    NHD ``[N, H, D]``.  ``key_lengths`` (int32 ``[B]`` on the device, ragged
    windows): entry b uses its first ``key_lengths[b]`` keys.  All buffers are
    carved from one workspace allocation.  Returns a dict with the workspace,
    the buffers' device addresses (``*_ptr``) and, with ``views``, tensor views
    ``ctiles`` ``[B, H, NCT, 2, 64 D]`` (block centroids), ``tiles``
    ``[B, H, NKB, 2, 64 D]`` and ``mean``/``var`` ``[B, H, D]`` (None without
    ``moments``); layouts per ``include/sol_attn_amd.h``.  The block tiles
    exist only when the keys do not qualify for rows mode (:func:`rows_mode`);
    otherwise the attention kernels read K and V themselves, which the dict
    keeps (``k``, ``v``).  ``qk_int8`` also quantises K per block
    (``sol_quantize_keys``) for the INT8-QK experiment.
    """
    lib = library()
    indexed = key_index is not None
    if indexed:
        b, tk = key_index.shape
        h, d = k.shape[-2:]
    else:
        b, tk, h, d = k.shape
    k, v = _rows(k), _rows(v)
    rows = not indexed and rows_mode(k, v, None, key_lengths)
    nkb = -(-tk // BLOCK)
    nct = -(-nkb // BLOCK)
    dev = k.device
    if stream is None:
        stream = _stream(dev)
    tile = 2 * BLOCK * d * 2  # bytes of one K/V tile pair
    sizes = [b * h * nct * tile, 0 if rows else b * h * nkb * tile]
    sizes += [b * h * -(-nkb // 16) * 2 * d * 4, b * h * d * 4, b * h * d * 4] if moments else [0, 0, 0]
    if qk_int8:
        sizes += [b * h * nkb * BLOCK * d, b * h * nkb * 4]
    offsets, total = _carve(tuple(sizes))
    ws = torch.empty(total, device=dev, dtype=torch.uint8)
    base = ws.data_ptr()
    ctiles, tiles = base + offsets[0], None if rows else base + offsets[1]
    sums, mean, var = (base + o for o in offsets[2:5]) if moments else (None, None, None)
    _check(lib.sol_pool_kv(k.data_ptr(), _strides(k, indexed), v.data_ptr(), _strides(v, indexed),
                           _ptr(key_index), _ptr(key_lengths), k.shape[0] if indexed else 0,
                           b, tk, h, d, ctiles, tiles, sums, mean, var, stream))
    pooled = {"workspace": ws, "shape": (b, h, d), "ctiles_ptr": ctiles, "tiles_ptr": tiles,
              "mean_ptr": mean, "var_ptr": var, "cov_ptr": None, "key_tokens": tk,
              "key_blocks": nkb, "key_lengths": key_lengths, "k8_ptr": None, "k8_scale_ptr": None,
              "k": k if rows else None, "v": v if rows else None}
    if qk_int8:
        k8, k8s = base + offsets[5], base + offsets[6]
        _check(lib.sol_quantize_keys(k.data_ptr(), _strides(k, indexed), _ptr(key_index), _ptr(key_lengths),
                                     k.shape[0] if indexed else 0, b, tk, h, d, int(rows), k8, k8s, stream))
        pooled["k8_ptr"], pooled["k8_scale_ptr"] = k8, k8s
        if views:
            pooled["k8_scale"] = _region(ws, offsets[6], torch.float32, (b, h, nkb))
    if views:
        pooled["ctiles"] = _region(ws, offsets[0], torch.bfloat16, (b, h, nct, 2, BLOCK * d))
        pooled["tiles"] = None if rows else _region(ws, offsets[1], torch.bfloat16, (b, h, nkb, 2, BLOCK * d))
        pooled["mean"] = _region(ws, offsets[3], torch.float32, (b, h, d)) if moments else None
        pooled["var"] = _region(ws, offsets[4], torch.float32, (b, h, d)) if moments else None
    return pooled


def key_covariance(pooled, stream=None):
    """Adds ``pooled["cov"]``: the full covariance of the key centroids, fp32
    ``[B, H, D, D]`` (``sol_key_covariance``), for the full-covariance
    threshold.  ``pooled`` must come from :func:`pool_kv` with moments."""
    if pooled["mean_ptr"] is None:
        raise ValueError("the full-covariance threshold needs the key moments (finite beta)")
    lib = library()
    b, h, d = pooled["shape"]
    dev = pooled["workspace"].device
    if stream is None:
        stream = _stream(dev)
    work = torch.empty(lib.sol_key_covariance_workspace_size(b, h, d) // 4, device=dev, dtype=torch.float32)
    cov = torch.empty((b, h, d, d), device=dev, dtype=torch.float32)
    _check(lib.sol_key_covariance(pooled["ctiles_ptr"], pooled["mean_ptr"], _ptr(pooled["key_lengths"]),
                                  b, pooled["key_tokens"], h, d, work.data_ptr(), cov.data_ptr(), stream))
    pooled["cov"] = cov
    pooled["cov_ptr"] = cov.data_ptr()
    return pooled


# Query blocks per SOL workgroup: 0 lets the library choose by launch size;
# 1 or 2 forces a form (results are bit-identical; the tests run both).
WORKGROUP_FORM = 0

# Pair query blocks by the stride sol_pair_strides picks (False: adjacent
# blocks share a workgroup).  Results are identical either way.
PAIRING = True
# Launches with fewer query blocks over all (entry, head) pairs are not
# paired: the three pairing kernels cost ~27 us, more than the union they
# save on a short attention launch.
PAIR_MIN_QUERY_BLOCKS = 8192


def _pair_buffers(q, rows, min_blocks):
    """``(q, workspace, strides, query_means)`` for a pairing launch, allocated
    on the current stream, or None when pairing does not apply (see
    :func:`pair_strides`).  ``query_means``: fp32 ``[B, H, NQB, D]``, the FP32
    query-block means the pairing pass also writes (the routing kernel's Qc)."""
    b, nq = rows.shape if rows is not None else q.shape[:2]
    h, d = q.shape[-2:]
    if b * h * -(-nq // BLOCK) < min_blocks:
        return None
    size = library().sol_pair_workspace_size(b, nq, h, d)
    if size == 0:
        return None
    return (_rows(q), torch.empty(size // 4, device=q.device, dtype=torch.float32),
            torch.empty((b, h), device=q.device, dtype=torch.int32),
            torch.empty((b, h, -(-nq // BLOCK), d), device=q.device, dtype=torch.float32))


def _pair_launch(q, rows, work, strides, means, stream):
    indexed = rows is not None
    b, nq = rows.shape if indexed else q.shape[:2]
    h, d = q.shape[-2:]
    _check(library().sol_pair_strides(q.data_ptr(), _strides(q, indexed), _ptr(rows),
                                      q.shape[0] if indexed else 0, b, nq, h, d,
                                      work.data_ptr(), strides.data_ptr(), _ptr(means), stream))


def _pairing(q, rows=None, stream=None):
    """``(strides, query_means)`` of a pairing launch on ``stream``, or
    ``(None, None)`` when pairing does not apply (:func:`pair_strides`)."""
    bufs = _pair_buffers(q, rows, PAIR_MIN_QUERY_BLOCKS)
    if bufs is None:
        return None, None
    qr, work, strides, means = bufs
    _pair_launch(qr, rows, work, strides, means, _stream(q.device) if stream is None else stream)
    return strides, means


def pair_strides(q, rows=None, min_blocks=None, stream=None):
    """Per-(entry, head) query-block pairing strides (int32 ``[B, H]``), or None
    when pairing does not apply: fewer than ``min_blocks`` query blocks in
    all (by default PAIR_MIN_QUERY_BLOCKS), or a sequence outside the
    library's 4 .. 8192 query blocks."""
    bufs = _pair_buffers(q, rows, PAIR_MIN_QUERY_BLOCKS if min_blocks is None else min_blocks)
    if bufs is None:
        return None
    qr, work, strides, _ = bufs
    _pair_launch(qr, rows, work, strides, None, _stream(q.device) if stream is None else stream)
    return strides


# Run the pairing kernels (they read Q only) on a second stream of the same
# device, concurrently with pooling (K and V only), joined back to the
# caller's stream before the attention launch.  False runs them on the
# caller's stream.  Results are identical either way.
OVERLAP_PAIRING = True
_side_streams = {}
_side_lock = threading.Lock()


def _side_stream(device, caller):
    """The side stream of one caller stream (``torch.cuda.Stream``) on
    ``device``, at the default priority.  Keyed by the caller's stream, so
    that calls issued concurrently on different streams (other threads, other
    streams of one thread) do not queue their pairing launches behind each
    other's."""
    key = (device.index, caller.cuda_stream)
    side = _side_streams.get(key)
    if side is None:
        with _side_lock:
            side = _side_streams.get(key)
            if side is None:
                side = _side_streams[key] = torch.cuda.Stream(device=device)
    return side


# Split the query-sink tiles of short launches over several workgroups
# (sol_split_workspace_size); False runs every tile in one workgroup.
SPLIT_SINKS = True


@functools.lru_cache(maxsize=256)
def _split_size(b, nq, nk, h, d, beta, q_sink):
    return library().sol_split_workspace_size(b, nq, nk, h, d, beta, q_sink)


@functools.lru_cache(maxsize=256)
def _pools_keys(b, nq, nk, h, d):
    return bool(library().sol_attention_pools_keys(b, nq, nk, h, d))


@functools.lru_cache(maxsize=256)
def _route_size(b, nq, nk, h, beta):
    return library().sol_route_workspace_size(b, nq, nk, h, beta)


# Route in a pre-pass kernel (sol_attention_fwd's route_workspace) when the
# pairing pass supplied the FP32 query-block means and the keys span at least
# ROUTE_MIN_CENTROID_TILES centroid tiles of 64 blocks; otherwise the
# attention kernel routes tile by tile as it streams the centroid tiles.
# The routing kernel saves that per-tile work and its barrier on long key
# sequences; short launches are latency-bound, and a second launch would
# cost more than it saves.  False never uses the routing kernel; "always"
# uses it for every launch at finite or +inf beta (forming the query means
# from Q when no pairing pass supplied them).  Decisions agree to the routing
# band either way.
ROUTE_PREPASS = True
ROUTE_MIN_CENTROID_TILES = 4


def route_workspace(b, nq, nk, h, beta, device):
    """The routing masks of an attention launch (None at beta = -inf)."""
    size = _route_size(b, nq, nk, h, float(beta))
    return torch.empty(size // 4, device=device, dtype=torch.int32) if size else None


def split_workspace(b, nq, nk, h, d, beta, q_sink, device):
    """The split workspace of an attention launch (None when it is not split)."""
    if not SPLIT_SINKS:
        return None
    size = _split_size(b, nq, nk, h, d, float(beta), int(q_sink))
    return torch.empty(size // 4, device=device, dtype=torch.float32) if size else None


_UNSET = object()


def attend(q, pooled, scale, beta, local, kv_sink, q_sink, protection=None, rows=None,
           debug=False, out=None, stats=True, stream=None, strides=_UNSET, query_means=None):
    """Routing + attention over pooled keys (the ``_sol`` launch of ``kernels.py:218-224``).

    ``pooled`` is the dict returned by :func:`pool_kv`.  ``rows`` (indexed
    windows) gathers the query rows.  With ``out`` (a contiguous BF16
    ``[N, H, D]`` tensor, indexed windows only) query i of window w is stored
    at ``out[rows[w, i]]`` instead of into a new ``[W, nq, H, D]`` tensor.
    ``strides``: pairing strides already computed (:func:`pair_strides`; None
    pairs adjacent blocks); by default they are computed here, with the
    query-block means.  ``query_means``: the FP32 query-block means of the
    pairing pass (``_pairing``), which let routing run as a pre-pass
    (ROUTE_PREPASS).
    Returns ``(out, counts, dbg)``; ``counts`` is None unless ``stats`` and
    ``dbg`` is None unless ``debug``.
    """
    lib = library()
    indexed = rows is not None
    b, h, d = pooled["shape"]
    nkb = pooled["key_blocks"]
    nq = rows.shape[1] if indexed else q.shape[1]
    nk = pooled["key_tokens"]
    q = _rows(q)
    dev = q.device
    if stream is None:
        stream = _stream(dev)
    nqb = -(-nq // BLOCK)
    scatter = out is not None
    if scatter:
        if not indexed or out.dtype != torch.bfloat16 or not out.is_contiguous() \
                or out.ndim != 3 or out.shape[1:] != (h, d) or out.device != dev:
            raise ValueError("out must be a contiguous BF16 [N, H, D] tensor on the Q device "
                             "(indexed windows only)")
    else:
        out = torch.empty((b, nq, h, d), device=dev, dtype=torch.bfloat16)
    counts = torch.empty((b, nqb, h), device=dev, dtype=torch.int32) if stats or debug else None
    dbg = None
    if debug:
        dbg = {"selected": torch.empty((b, nqb, h, nkb), device=dev, dtype=torch.uint8),
               "proxy": torch.full((b, nqb, h, nkb), math.nan, device=dev, dtype=torch.float32),
               "cutoff": torch.empty((b, nqb, h), device=dev, dtype=torch.float32)}
    prot = None
    if protection is not None:
        prot = protection.contiguous().view(torch.uint8)
    if strides is _UNSET:
        strides, query_means = _pairing(q, rows, stream) if PAIRING else (None, None)
    split = split_workspace(b, nq, nk, h, d, beta, q_sink, dev)
    route = None
    if beta != -math.inf and (ROUTE_PREPASS == "always" or (
            ROUTE_PREPASS and query_means is not None and -(-nkb // BLOCK) >= ROUTE_MIN_CENTROID_TILES)):
        route = route_workspace(b, nq, nk, h, beta, dev)
    else:
        query_means = None
    kr, vr = pooled["k"], pooled["v"]
    _check(lib.sol_attention_fwd(
        q.data_ptr(), _strides(q, indexed), _ptr(rows), q.shape[0] if indexed else 0,
        b, nq, nk, _ptr(pooled["key_lengths"]), h, d,
        _ptr(kr), None if kr is None else _strides(kr), _ptr(vr), None if vr is None else _strides(vr),
        pooled["tiles_ptr"], pooled["ctiles_ptr"], pooled["mean_ptr"], pooled["var_ptr"], pooled["cov_ptr"],
        _ptr(prot), _ptr(strides), _ptr(split), _ptr(route), _ptr(query_means), float(scale), float(beta),
        int(local), int(kv_sink), int(q_sink),
        out.data_ptr(), _ptr(rows if scatter else None), _ptr(counts),
        _ptr(dbg and dbg["selected"]), _ptr(dbg and dbg["proxy"]), _ptr(dbg and dbg["cutoff"]),
        pooled["k8_ptr"], pooled["k8_scale_ptr"], WORKGROUP_FORM, stream))
    if debug:
        dbg["selected"] = dbg["selected"].bool()
    return out, counts, dbg


# Short launches over at most 16 key blocks pool the keys inside the
# attention launch (sol_attention_pools_keys): the whole call is one kernel.
# False always runs the pooling kernel first.  Results are identical either
# way (the same centroids and moments, bit for bit).
SELF_POOLING = True

# Plain BTHD calls that need no query-block pairing go through one C-ABI call,
# sol_attention_all_in (pooling + attention, the pooled key buffers carved
# from one workspace), instead of sol_pool_kv + sol_attention_fwd: the same
# kernels and workspace layout, bit-identical results, and one call's host
# cost fewer.  False keeps the two calls.
ALL_IN = True


@functools.lru_cache(maxsize=256)
def _all_in_size(b, nq, nk, h, d, beta, q_sink, k_stride, v_stride):
    return library().sol_attention_workspace_size(b, nq, nk, h, d, beta, q_sink, k_stride, v_stride)


def _all_in(q, k, v, scale, beta, local, kv_sink, q_sink, stats):
    """``(out, counts)`` of one sol_attention_all_in call (BTHD, the caller's stream)."""
    q, k, v = _rows(q), _rows(k), _rows(v)
    b, nq, h, d = q.shape
    nk = k.shape[1]
    dev = q.device
    size = _all_in_size(b, nq, nk, h, d, beta, q_sink, k.stride(1), v.stride(1))
    if size < 0:
        raise RuntimeError("sol_attention_workspace_size rejected the sizes")
    ws = torch.empty(size, device=dev, dtype=torch.uint8) if size else None
    out = torch.empty((b, nq, h, d), device=dev, dtype=torch.bfloat16)
    counts = torch.empty((b, -(-nq // BLOCK), h), device=dev, dtype=torch.int32) if stats else None
    _check(library().sol_attention_all_in(
        q.data_ptr(), _strides(q), k.data_ptr(), _strides(k), v.data_ptr(), _strides(v), b, nq, nk, h, d,
        scale, beta, local, kv_sink, q_sink, _ptr(ws), size, out.data_ptr(), _ptr(counts), _stream(dev)))
    return out, counts


def _self_pooled(k, v):
    """The ``pool_kv`` record of keys the attention launch pools itself: plain
    K / V rows and no pooled buffers."""
    k, v = _rows(k), _rows(v)
    b, nk, h, d = k.shape
    return {"workspace": None, "shape": (b, h, d), "ctiles_ptr": None, "tiles_ptr": None,
            "mean_ptr": None, "var_ptr": None, "cov_ptr": None, "key_tokens": nk,
            "key_blocks": -(-nk // BLOCK), "key_lengths": None, "k8_ptr": None, "k8_scale_ptr": None,
            "k": k, "v": v}


def launch_sol(q, k, v, scale, beta, local, kv_sink, q_sink, stats, protection=None,
               rows=None, keys=None, debug=False, key_lengths=None, out=None,
               threshold_estimator="diagonal_covariance", qk_precision="bf16"):
    """All-in SOL attention (``kernels.py:203-225``): pooling, moments, routing, attention.

    ``rows``/``keys`` (indexed windows) gather Q and K/V token rows inside the
    kernels instead of materialising copies; ``key_lengths`` makes the windows'
    key counts ragged and ``out`` scatters the result rows (see :func:`attend`).
    ``threshold_estimator="full_covariance"`` builds the cutoff from the full
    key covariance (:func:`key_covariance`) instead of its diagonal;
    ``qk_precision="int8"`` runs the exact blocks' scores on INT8 (queries
    per row, keys per block; the INT8-QK experiment).
    Returns ``(out, counts)`` (``counts`` None unless ``stats``) and, with
    ``debug=True``, a dict of routing diagnostics as a third element.

    ``beta = -inf`` selects every key block: for plain BTHD inputs (no index,
    protection, scatter or diagnostics) that is exact attention over all keys,
    which the dense kernel computes with the same per-query tile order and
    arithmetic (bit-identical output), without the pooling pass.  A forced
    WORKGROUP_FORM keeps it on the SOL kernel.
    """
    if (beta == -math.inf and WORKGROUP_FORM == 0 and rows is None and keys is None and protection is None
            and key_lengths is None and out is None and not debug and qk_precision == "bf16"):
        b, nq, h = q.shape[0], q.shape[1], q.shape[2]
        dense = launch_dense(q, k, v, scale)
        counts = None
        if stats:
            counts = torch.full((b, -(-nq // BLOCK), h), -(-k.shape[1] // BLOCK), device=q.device, dtype=torch.int32)
        return dense, counts
    plain = (rows is None and keys is None and key_lengths is None and not debug and qk_precision == "bf16"
             and threshold_estimator == "diagonal_covariance" and WORKGROUP_FORM == 0
             and ROUTE_PREPASS != "always")
    if (ALL_IN and plain and protection is None and out is None and SELF_POOLING and SPLIT_SINKS
            and (not PAIRING or q.shape[0] * q.shape[2] * -(-q.shape[1] // BLOCK) < PAIR_MIN_QUERY_BLOCKS)):
        # No pairing pass: pooling and attention in one C-ABI call.
        return _all_in(q, k, v, float(scale), float(beta), int(local), int(kv_sink), int(q_sink), stats)
    stream = _stream(q.device)
    if (SELF_POOLING and plain and rows_mode(k, v)
            and _pools_keys(q.shape[0], q.shape[1], k.shape[1], q.shape[2], q.shape[3])):
        # One launch: the attention kernel pools the keys itself.
        out, counts, _ = attend(q, _self_pooled(k, v), scale, beta, local, kv_sink, q_sink, protection,
                                out=out, stats=stats, stream=stream, strides=None)
        return out, counts
    strides, pairing, means = _UNSET, None, None
    if PAIRING and OVERLAP_PAIRING:
        # Buffers come from the caller's stream and stay referenced until the
        # join below, so no other allocation can reuse them while the side
        # stream still works on them.
        pairing = _pair_buffers(q, rows, PAIR_MIN_QUERY_BLOCKS)
        strides = None
        if pairing is not None:
            main = torch.cuda.current_stream(q.device)
            side = _side_stream(q.device, main)
            side.wait_stream(main)
            try:
                _pair_launch(pairing[0], rows, pairing[1], pairing[2], pairing[3], side.cuda_stream)
            except BaseException:
                main.wait_stream(side)
                raise
            strides, means = pairing[2], pairing[3]
    try:
        pooled = pool_kv(k, v, key_index=keys, moments=not math.isinf(beta), key_lengths=key_lengths,
                         stream=stream, views=debug, qk_int8=qk_precision == "int8")
        if threshold_estimator == "full_covariance" and not math.isinf(beta):
            key_covariance(pooled, stream)
    finally:
        # Joined on every path: an error above must not leave the pairing
        # buffers free for reuse while the side stream still writes them.
        if pairing is not None:
            main.wait_stream(side)
    out, counts, dbg = attend(q, pooled, scale, beta, local, kv_sink, q_sink, protection, rows,
                              debug, out, stats, stream, strides=strides, query_means=means)
    del pairing
    if debug:
        dbg.update(pooled)
        return out, counts, dbg
    return out, counts


def plan_protection(rows, keys, key_lengths, local_tokens, ranges):
    """Packed-block protection of indexed windows on the GPU (``sol_plan_protection``).

    ``rows`` ``[W, nq]`` / ``keys`` ``[W, nk]`` int64, ``key_lengths`` int32
    ``[W]`` or None, all validated and on one GPU; ``ranges``: sequence of
    ``(a, b)``.  Returns bool ``[W, NQB, NKB]``.
    """
    lib = library()
    dev = rows.device
    rows, keys = rows.contiguous(), keys.contiguous()
    w, nq = rows.shape
    nk = keys.shape[1]
    out = torch.empty((w, -(-nq // BLOCK), -(-nk // BLOCK)), device=dev, dtype=torch.uint8)
    rng = torch.tensor(list(ranges), dtype=torch.int64).reshape(-1, 2).to(dev) if ranges else None
    _check(lib.sol_plan_protection(rows.data_ptr(), keys.data_ptr(), _ptr(key_lengths),
                                   w, nq, nk, int(local_tokens), _ptr(rng),
                                   0 if rng is None else rng.shape[0], out.data_ptr(), _stream(dev)))
    return out.view(torch.bool)


def launch_dense(q, k, v, scale, rows=None, out=None):
    """Dense control (``kernels.py:193-200``): non-causal attention over all keys.

    ``rows`` (int64 ``[W, nq]`` on the Q device): Q is NHD ``[N, H, D]`` and
    query i of window w is Q row ``rows[w, i]``, gathered inside the kernel;
    K / V (NHD ``[nk, H, D]``) are the keys every window attends.  With
    ``out`` (a contiguous BF16 ``[N, H, D]`` tensor) that query's result is
    stored at ``out[rows[w, i]]`` and ``out`` is returned -- the
    ``out[rows] = dense(q[rows], k, v)`` of a window adapter's anchor-row and
    global queries (``integrations/vdn.py:57-61``) in one launch, without
    gathered copies; otherwise a new ``[W, nq, H, D]`` tensor.
    """
    lib = library()
    q, k, v = _rows(q), _rows(k), _rows(v)
    indexed = rows is not None
    if indexed:
        if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
            raise ValueError("indexed dense attention takes NHD Q/K/V")
        rows = rows.contiguous()
        w, nq = rows.shape
        k, v = k.unsqueeze(0), v.unsqueeze(0)
        b, n, (h, d) = 1, q.shape[0], q.shape[1:]
        tq = w * nq
    else:
        if out is not None:
            raise ValueError("out= needs rows")
        b, tq, h, d = q.shape
    nk = k.shape[1]
    scatter = out is not None
    if scatter:
        if out.dtype != torch.bfloat16 or not out.is_contiguous() or out.shape != q.shape or out.device != q.device:
            raise ValueError("out must be a contiguous BF16 tensor shaped like Q on its device")
    else:
        out = torch.empty((w, nq, h, d) if indexed else (b, tq, h, d), device=q.device, dtype=torch.bfloat16)
    tiles = None if rows_mode(k, v) else _tiles(b, h, -(-nk // BLOCK), d, q.device)
    _check(lib.sol_dense_fwd(q.data_ptr(), _strides(q, indexed), _ptr(rows), n if indexed else 0,
                             k.data_ptr(), _strides(k), v.data_ptr(), _strides(v),
                             b, tq, nk, h, d, float(scale), _ptr(tiles), out.data_ptr(),
                             _ptr(rows if scatter else None), _stream(q.device)))
    return out
