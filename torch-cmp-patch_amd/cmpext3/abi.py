"""ctypes binding of the C ABI in include/cmpext3_attn.h, for torch tensors.

This is the FFI stub a host program written in Python would use to call the
library directly (the torch extension `cmpext3._native` is the other caller).
The library is loaded from this package directory; loading it needs no GPU.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcmpext3_attn.so")

# Every function include/cmpext3_attn.h declares.
SYMBOLS = ("cmpext3_attn_fwd", "cmpext3_attn_fwd_gqa", "cmpext3_attn_fwd_masked",
           "cmpext3_attn_fwd_ws", "cmpext3_attn_fwd_workspace_size", "cmpext3_attn_fwd_plan",
           "cmpext3_attn_fwd_noalloc", "cmpext3_attn_fwd_lse", "cmpext3_attn_bwd",
           "cmpext3_attn_bwd_ws", "cmpext3_attn_bwd_workspace_size",
           "cmpext3_attn_strerror", "cmpext3_attn_abi_version", "cmpext3_attn_describe")

DTYPE_F16, DTYPE_BF16, DTYPE_F32, DTYPE_BOOL = 0, 1, 2, 3
WORKSPACE_COUNTER_BYTES = 65536                     # CMPEXT3_WORKSPACE_COUNTER_BYTES
NOALLOC_SCRATCH_BYTES = 65536 + 16 * 1024 * 1024    # CMPEXT3_NOALLOC_SCRATCH_BYTES
(OK, E_INVALID, E_DTYPE, E_HEAD_DIM, E_ALIGN, E_EMPTY_KEYS, E_LAUNCH, E_TOO_LARGE, E_MASK,
 E_TRAINING) = range(10)

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built (python torch-cmp-patch_amd/build.py)")
        L = ctypes.CDLL(LIB_PATH)
        i64p = ctypes.POINTER(ctypes.c_int64)
        vp = ctypes.c_void_p
        ci = ctypes.c_int
        L.cmpext3_attn_fwd.argtypes = [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci,
                                       i64p, i64p, i64p, i64p, ctypes.c_float, ci, vp]
        L.cmpext3_attn_fwd.restype = ci
        L.cmpext3_attn_fwd_gqa.argtypes = [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci,
                                           i64p, i64p, i64p, i64p, ctypes.c_float, ci, vp]
        L.cmpext3_attn_fwd_gqa.restype = ci
        L.cmpext3_attn_fwd_masked.argtypes = [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci,
                                              i64p, i64p, i64p, i64p, vp, ci, i64p,
                                              ctypes.c_float, ci, vp]
        L.cmpext3_attn_fwd_masked.restype = ci
        L.cmpext3_attn_fwd_noalloc.argtypes = L.cmpext3_attn_fwd_masked.argtypes
        L.cmpext3_attn_fwd_noalloc.restype = ci
        sz = ctypes.c_size_t
        L.cmpext3_attn_fwd_ws.argtypes = [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci,
                                          i64p, i64p, i64p, i64p, vp, ci, i64p,
                                          ctypes.c_float, ci, vp, sz, vp]
        L.cmpext3_attn_fwd_ws.restype = ci
        L.cmpext3_attn_fwd_workspace_size.argtypes = [ci] * 10
        L.cmpext3_attn_fwd_workspace_size.restype = sz
        L.cmpext3_attn_fwd_plan.argtypes = [ci] * 10 + [sz, ctypes.POINTER(ci)]
        L.cmpext3_attn_fwd_plan.restype = ci
        L.cmpext3_attn_fwd_lse.argtypes = [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci,
                                           i64p, i64p, i64p, i64p, vp, ci, i64p, ctypes.c_float, ci,
                                           vp, sz, vp]
        L.cmpext3_attn_fwd_lse.restype = ci
        L.cmpext3_attn_bwd.argtypes = ([vp] * 10 + [ci] * 7 + [i64p] * 8 + [vp, ci, i64p]
                                       + [ctypes.c_float, ci, vp])
        L.cmpext3_attn_bwd.restype = ci
        L.cmpext3_attn_bwd_ws.argtypes = ([vp] * 10 + [ci] * 7 + [i64p] * 8 + [vp, ci, i64p]
                                          + [ctypes.c_float, ci, vp, sz, vp])
        L.cmpext3_attn_bwd_ws.restype = ci
        L.cmpext3_attn_bwd_workspace_size.argtypes = [ci] * 9
        L.cmpext3_attn_bwd_workspace_size.restype = sz
        L.cmpext3_attn_strerror.argtypes = [ci]
        L.cmpext3_attn_strerror.restype = ctypes.c_char_p
        L.cmpext3_attn_abi_version.argtypes = []
        L.cmpext3_attn_abi_version.restype = ci
        L.cmpext3_attn_describe.argtypes = [ci, ci, ci, ci, ci, ci, ci, ctypes.c_char_p, ci]
        L.cmpext3_attn_describe.restype = ci
        _lib = L
    return _lib


def strerror(code: int) -> str:
    return lib().cmpext3_attn_strerror(code).decode()


def describe(dtype: int, B: int, H: int, Sq: int, Sk: int, D: int, causal: bool = False):
    buf = ctypes.create_string_buffer(384)
    rc = lib().cmpext3_attn_describe(dtype, B, H, Sq, Sk, D, int(causal), buf, 384)
    return rc, buf.value.decode()


def workspace_size(dtype: int, B: int, H: int, Hkv: int, Sq: int, Sk: int, D: int,
                   mask_dtype: int = -1, causal: bool = False, with_lse: bool = False) -> int:
    """Bytes of workspace the full key-split plan of this problem takes (host only)."""
    return lib().cmpext3_attn_fwd_workspace_size(dtype, B, H, Hkv, Sq, Sk, D, mask_dtype,
                                                 int(causal), int(with_lse))


def plan(dtype: int, B: int, H: int, Hkv: int, Sq: int, Sk: int, D: int, workspace_bytes: int,
         mask_dtype: int = -1, causal: bool = False, with_lse: bool = False):
    """(return code, key ranges per split block) a launch takes with this much
    workspace (host only; 1 = unsplit)."""
    parts = ctypes.c_int(-1)
    rc = lib().cmpext3_attn_fwd_plan(dtype, B, H, Hkv, Sq, Sk, D, mask_dtype, int(causal),
                                     int(with_lse), workspace_bytes, ctypes.byref(parts))
    return rc, parts.value


# Key-split workspaces of (device, stream), as the torch binding keeps them:
# zero-filled byte tensors (the counters must start at zero; every launch
# leaves them so), grown on demand, reused by the calls on that stream.
_workspaces: dict = {}


def workspace_for(t, handle: int, need: int):
    """(pointer, bytes) of the workspace for stream `handle` on t's device, at
    least `need` bytes; (None, 0) under graph capture or when need is 0."""
    import torch
    if need == 0 or torch.cuda.is_current_stream_capturing():
        return None, 0
    key = (t.device.index, handle)
    w = _workspaces.get(key)
    if w is None or w.numel() < need:
        w = torch.zeros(need, dtype=torch.uint8, device=t.device)
        _workspaces[key] = w
    return w.data_ptr(), w.numel()


def dtype_code(dtype) -> int:
    import torch
    return {torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32,
            torch.bool: DTYPE_BOOL}[dtype]


def prepare_mask(mask, B: int, H: int, Sq: int, Sk: int, runs: bool = False):
    """attn_mask broadcast to [B,H,Sq,Sk] in a layout the C ABI takes: a view
    when the given tensor has a unit key stride (inference calls read any
    other layout element by element), else a compact copy.  runs=True (the
    training entry points) also needs rows readable in runs of 8 keys: other
    strides multiples of 4 elements, Sk a multiple of 8, 16-byte aligned
    base; the copy's rows are zero-padded to a multiple of 8."""
    import torch
    m = mask.expand(B, H, Sq, Sk)
    fits = m.stride(3) == 1 and (not runs or (Sk % 8 == 0 and all(m.stride(i) % 4 == 0 for i in range(3))
                                              and m.data_ptr() % 16 == 0))
    if not fits:
        cb, ch, cq = (1 if m.stride(0) == 0 else B), (1 if m.stride(1) == 0 else H), \
                     (1 if m.stride(2) == 0 else Sq)
        c = torch.zeros(cb, ch, cq, (Sk + 7) // 8 * 8, dtype=m.dtype, device=m.device)
        c[..., :Sk].copy_(m[:cb, :ch, :cq])
        m = c[..., :Sk].expand(B, H, Sq, Sk)
    return m


def _strides(t):
    arr = (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))
    return arr


def attn_fwd_raw(q, k, v, o, scale: float, causal: bool = False, stream=None,
                 D: Optional[int] = None, attn_mask=None, workspace=True) -> int:
    """Call cmpext3_attn_fwd_ws on [B,H,S,D] tensors (any strides with unit last
    stride; k/v may hold fewer heads than q: grouped-query) with this module's
    workspace for the stream (workspace=True), a given uint8 device tensor
    (zeroed before its first use), or none (workspace=False: no key split;
    with no mask the plain cmpext3_attn_fwd / _gqa entry points are called).
    Returns the C return code; launches on `stream` (a torch.cuda.Stream, a raw
    handle, or None for the current stream)."""
    import torch
    if stream is None:
        handle = torch.cuda.current_stream(q.device).cuda_stream if q.is_cuda else 0
    elif isinstance(stream, int):
        handle = stream
    else:
        handle = stream.cuda_stream
    B, H, Sq, Dq = q.shape
    Dx = Dq if D is None else D
    ptrs = (ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()),
            ctypes.c_void_p(v.data_ptr()), ctypes.c_void_p(o.data_ptr()))
    strides = (_strides(q), _strides(k), _strides(v), _strides(o))
    dt = dtype_code(q.dtype)
    if workspace is False and attn_mask is None:
        tail = (*strides, ctypes.c_float(scale), int(causal), ctypes.c_void_p(handle))
        if k.shape[1] != H:
            return lib().cmpext3_attn_fwd_gqa(*ptrs, dt, B, H, k.shape[1], Sq, k.shape[2], Dx, *tail)
        return lib().cmpext3_attn_fwd(*ptrs, dt, B, H, Sq, k.shape[2], Dx, *tail)
    mp, mdt, mst, _keep = _mask_args(attn_mask, B, H, Sq, k.shape[2])
    wp, wb = None, 0
    if workspace is True and q.is_cuda:
        wp, wb = workspace_for(q, handle, workspace_size(dt, B, H, k.shape[1], Sq, k.shape[2], Dx,
                                                         mdt, causal))
    elif workspace is not False and workspace is not None:
        wp, wb = workspace.data_ptr(), workspace.numel()
    return lib().cmpext3_attn_fwd_ws(*ptrs, dt, B, H, k.shape[1], Sq, k.shape[2], Dx, *strides,
                                     mp, mdt, mst, ctypes.c_float(scale), int(causal),
                                     ctypes.c_void_p(wp), wb, ctypes.c_void_p(handle))


def attn_fwd_noalloc_raw(q, k, v, o, scale: float, causal: bool = False, stream=None,
                         attn_mask=None) -> int:
    """Call cmpext3_attn_fwd_noalloc (the allocation-free forward) on
    caller-allocated tensors; k/v may hold fewer heads than q.  Returns the C
    return code."""
    B, H, Sq, D = q.shape
    mp, mdt, mst, _keep = _mask_args(attn_mask, B, H, Sq, k.shape[2])
    vp = ctypes.c_void_p
    return lib().cmpext3_attn_fwd_noalloc(
        *(vp(t.data_ptr()) for t in (q, k, v, o)), dtype_code(q.dtype), B, H, k.shape[1], Sq,
        k.shape[2], D, _strides(q), _strides(k), _strides(v), _strides(o), mp, mdt, mst,
        ctypes.c_float(scale), int(causal), vp(_handle(q, stream)))


def attn_fwd(q, k, v, scale: Optional[float] = None, causal: bool = False, stream=None,
             attn_mask=None):
    """Allocate O like q (contiguous [B,H,Sq,D]) and run the kernel through the C ABI.
    Raises RuntimeError with the library's message on a non-zero return code."""
    import torch
    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    rc = attn_fwd_raw(q, k, v, o, scale, causal, stream, attn_mask=attn_mask)
    if rc != OK:
        raise RuntimeError(f"cmpext3_attn_fwd: {strerror(rc)} (code {rc})")
    return o


def _handle(t, stream):
    import torch
    if stream is None:
        return torch.cuda.current_stream(t.device).cuda_stream
    return stream if isinstance(stream, int) else stream.cuda_stream


def _mask_args(attn_mask, B, H, Sq, Sk, runs=False):
    """(pointer, dtype code, strides, keep-alive tensor) for an optional mask."""
    if attn_mask is None:
        return ctypes.c_void_p(0), -1, (ctypes.c_int64 * 3)(0, 0, 0), None
    m = prepare_mask(attn_mask, B, H, Sq, Sk, runs)
    return (ctypes.c_void_p(m.data_ptr()), dtype_code(m.dtype),
            (ctypes.c_int64 * 3)(m.stride(0), m.stride(1), m.stride(2)), m)


def attn_fwd_lse(q, k, v, scale: Optional[float] = None, causal: bool = False, stream=None,
                 attn_mask=None, workspace: bool = True):
    """Training forward through cmpext3_attn_fwd_lse: returns (O, lse) with
    lse the fp32 [B,H,Sq] natural-log row log-sum-exp (k, v may hold fewer
    heads than q: grouped-query); workspace=False passes none (no key split).
    Raises RuntimeError on a non-zero code."""
    import torch
    B, H, Sq, D = q.shape
    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, H, Sq, dtype=torch.float32, device=q.device)
    if scale is None:
        scale = D ** -0.5
    mp, mdt, mst, _keep = _mask_args(attn_mask, B, H, Sq, k.shape[2], runs=True)
    handle = _handle(q, stream)
    wp, wb = workspace_for(q, handle, workspace_size(dtype_code(q.dtype), B, H, k.shape[1], Sq,
                                                     k.shape[2], D, mdt, causal, with_lse=True)) \
        if workspace else (None, 0)
    rc = lib().cmpext3_attn_fwd_lse(
        ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()),
        ctypes.c_void_p(o.data_ptr()), ctypes.c_void_p(lse.data_ptr()), dtype_code(q.dtype),
        B, H, k.shape[1], Sq, k.shape[2], D, _strides(q), _strides(k), _strides(v), _strides(o),
        mp, mdt, mst, ctypes.c_float(scale), int(causal), ctypes.c_void_p(wp), wb,
        ctypes.c_void_p(handle))
    if rc != OK:
        raise RuntimeError(f"cmpext3_attn_fwd_lse: {strerror(rc)} (code {rc})")
    return o, lse


def bwd_workspace_size(dtype: int, B: int, H: int, H_kv: int, Sq: int, Sk: int, D: int,
                       mask_dtype: int = -1, causal: bool = False) -> int:
    """cmpext3_attn_bwd_workspace_size: bytes that let the backward split its
    gradient sweeps (0 = it never splits)."""
    return lib().cmpext3_attn_bwd_workspace_size(dtype, B, H, H_kv, Sq, Sk, D, mask_dtype, int(causal))


def attn_bwd_raw(q, k, v, o, do, lse, dq, dk, dv, delta, scale: float, causal: bool = False,
                 stream=None, attn_mask=None, workspace=None) -> int:
    """Call cmpext3_attn_bwd (workspace None) or cmpext3_attn_bwd_ws (a byte
    tensor, or True for one of cmpext3_attn_bwd_workspace_size bytes made
    here) on caller-allocated tensors; returns the C code."""
    B, H, Sq, D = q.shape
    vp = ctypes.c_void_p
    mp, mdt, mst, _keep = _mask_args(attn_mask, B, H, Sq, k.shape[2], runs=True)
    args = [*(vp(t.data_ptr()) for t in (q, k, v, o, do, lse, dq, dk, dv, delta)),
            dtype_code(q.dtype), B, H, k.shape[1], Sq, k.shape[2], D,
            *(_strides(t) for t in (q, k, v, o, do, dq, dk, dv)),
            mp, mdt, mst, ctypes.c_float(scale), int(causal)]
    if workspace is None:
        return lib().cmpext3_attn_bwd(*args, vp(_handle(q, stream)))
    if workspace is True:
        import torch
        n = bwd_workspace_size(dtype_code(q.dtype), B, H, k.shape[1], Sq, k.shape[2], D, mdt, causal)
        workspace = torch.empty(max(n, 16), dtype=torch.uint8, device=q.device)
    return lib().cmpext3_attn_bwd_ws(*args, vp(workspace.data_ptr()), workspace.numel(),
                                     vp(_handle(q, stream)))


def attn_bwd(q, k, v, o, do, lse, scale: Optional[float] = None, causal: bool = False, stream=None,
             attn_mask=None, workspace=True):
    """Gradients (dq, dk, dv) through cmpext3_attn_bwd_ws (outputs contiguous;
    the delta workspace and, with workspace=True, the split workspace
    allocated here; workspace=None: cmpext3_attn_bwd, never split).  Raises
    RuntimeError on a non-zero code."""
    import torch
    B, H, Sq, D = q.shape
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    delta = torch.empty(B, H, Sq, dtype=torch.float32, device=q.device)
    if scale is None:
        scale = D ** -0.5
    rc = attn_bwd_raw(q, k, v, o, do, lse, dq, dk, dv, delta, scale, causal, stream, attn_mask, workspace)
    if rc != OK:
        raise RuntimeError(f"cmpext3_attn_bwd: {strerror(rc)} (code {rc})")
    return dq, dk, dv
