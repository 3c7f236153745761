"""ctypes view of the C ABI in include/ifa4.h (libifa4.so).

Used for host-only queries (tile table, tile counts, argument validation) and
by tests that call the library directly.  The compute path goes through the
torch binding (`_native.py`), which calls the same library.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# Same override as the torch binding loader (_native.py): a sweep variant directory.
LIB_PATH = os.path.join(os.environ.get("IFA4_LIB_DIR", _HERE), "libifa4.so")

IFA4_OK = 0
IFA4_EINVAL = 1
IFA4_EUNSUPPORTED = 2
IFA4_EWORKSPACE = 3
IFA4_ELAUNCH = 4

IFA4_BF16 = 0
IFA4_FP16 = 1
IFA4_FP32 = 2
IFA4_FP8_E4M3 = 3

IFA4_FLAG_NO_PRUNE = 0x1
IFA4_FLAG_BOTTOM_RIGHT = 0x2
IFA4_FLAG_SPLIT_KV_2 = 0x4

# Every function include/ifa4.h declares: name -> (restype, argtypes).
_c_int32 = ctypes.c_int32
_c_int64 = ctypes.c_int64
_vp = ctypes.c_void_p


class Ifa4Args(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("q", _vp), ("k", _vp), ("v", _vp), ("rel", _vp),
        ("out", _vp), ("lse", _vp),
        ("cu_seqlens_q", _vp), ("cu_seqlens_k", _vp),
        ("q_stride_t", _c_int64), ("q_stride_h", _c_int64),
        ("k_stride_t", _c_int64), ("k_stride_h", _c_int64),
        ("v_stride_t", _c_int64), ("v_stride_h", _c_int64),
        ("rel_stride_t", _c_int64), ("rel_stride_h", _c_int64),
        ("out_stride_t", _c_int64), ("out_stride_h", _c_int64),
        ("lse_stride_h", _c_int64),
        ("total_q", _c_int64), ("total_k", _c_int64),
        ("batch", _c_int32), ("n_heads", _c_int32), ("kv_heads", _c_int32),
        ("head_dim", _c_int32), ("rel_extent", _c_int32), ("rel_width", _c_int32),
        ("max_seqlen_q", _c_int32), ("max_seqlen_k", _c_int32),
        ("window_left", _c_int32), ("causal", _c_int32),
        ("softmax_scale", ctypes.c_float),
        ("qkv_dtype", _c_int32), ("rel_dtype", _c_int32),
    ]


class Ifa4Tile(ctypes.Structure):
    _fields_ = [("block_q", _c_int32), ("block_k", _c_int32), ("waves", _c_int32),
                ("stages", _c_int32), ("kv_chunk", _c_int32)]


class Ifa4PagedKV(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32), ("block_size", _c_int32),
        ("block_table", _vp), ("seqused_k", _vp),
        ("block_table_stride", _c_int64), ("k_stride_block", _c_int64),
        ("v_stride_block", _c_int64),
        ("num_blocks", _c_int32), ("max_blocks_per_seq", _c_int32),
    ]


class Ifa4KvQuant(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("kv_dtype", _c_int32),
                ("k_scale", ctypes.c_float), ("v_scale", ctypes.c_float)]


class Ifa4RelProj(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("d_rel", _c_int32), ("r", _vp),
                ("r_stride_t", _c_int64), ("r_stride_h", _c_int64), ("wt", _vp)]


_P_ARGS = ctypes.POINTER(Ifa4Args)
_P_PAGED = ctypes.POINTER(Ifa4PagedKV)
_P_QUANT = ctypes.POINTER(Ifa4KvQuant)
_P_TILE = ctypes.POINTER(Ifa4Tile)
_P_I32 = ctypes.POINTER(ctypes.c_int32)
_P_I64 = ctypes.POINTER(ctypes.c_int64)

SIGNATURES = {
    "ifa4_status_str": (ctypes.c_char_p, [_c_int32]),
    "ifa4_abi_version": (_c_int32, []),
    "ifa4_validate": (_c_int32, [_P_ARGS]),
    "ifa4_prefill_fwd": (_c_int32, [_P_ARGS, _vp]),
    "ifa4_prefill_workspace_bytes": (ctypes.c_size_t, [_P_ARGS]),
    "ifa4_prefill_fwd_ws": (_c_int32, [_P_ARGS, _vp, ctypes.c_size_t, _vp]),
    "ifa4_prefill_tile": (_c_int32, [_P_ARGS, _P_TILE]),
    "ifa4_prefill_rproj_fwd": (_c_int32, [_P_ARGS, ctypes.POINTER(Ifa4RelProj), _vp]),
    "ifa4_prefill_count_tiles": (_c_int32, [_P_ARGS, _P_I32, _P_I32, _P_I64, _P_I64]),
    "ifa4_decode_workspace_bytes": (ctypes.c_size_t, [_P_ARGS]),
    "ifa4_decode_tile": (_c_int32, [_P_ARGS, _P_TILE]),
    "ifa4_decode_fwd": (_c_int32, [_P_ARGS, _vp, ctypes.c_size_t, _vp]),
    "ifa4_decode_fwd_noalloc": (_c_int32, [_P_ARGS, _vp]),
    "ifa4_decode_paged_workspace_bytes": (ctypes.c_size_t, [_P_ARGS, _P_PAGED]),
    "ifa4_decode_paged_fwd": (_c_int32, [_P_ARGS, _P_PAGED, _vp, ctypes.c_size_t, _vp]),
    "ifa4_decode_quant_workspace_bytes": (ctypes.c_size_t, [_P_ARGS, _P_PAGED, _P_QUANT]),
    "ifa4_decode_quant_fwd": (_c_int32, [_P_ARGS, _P_PAGED, _P_QUANT, _vp, ctypes.c_size_t,
                                         _vp]),
}

_lib = None


def lib():
    """Load libifa4.so once; raise ImportError with the build hint if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing; build it with "
                "`python inkling-fa4-relative-attention_amd/build.py`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, argt) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = argt
        _lib = handle
    return _lib


def status_str(code):
    return lib().ifa4_status_str(code).decode()


def make_args(**kw):
    """Ifa4Args with struct_size filled and sane defaults, overridden by kw."""
    a = Ifa4Args()
    a.struct_size = ctypes.sizeof(Ifa4Args)
    a.window_left = -1
    a.causal = 1
    a.softmax_scale = 1.0
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def make_paged(**kw):
    """Ifa4PagedKV with struct_size filled, fields from kw."""
    kv = Ifa4PagedKV()
    kv.struct_size = ctypes.sizeof(Ifa4PagedKV)
    for k, v in kw.items():
        setattr(kv, k, v)
    return kv


def make_quant(**kw):
    """Ifa4KvQuant with struct_size filled (fp8 e4m3, scales 1), fields from kw."""
    qt = Ifa4KvQuant()
    qt.struct_size = ctypes.sizeof(Ifa4KvQuant)
    qt.kv_dtype = IFA4_FP8_E4M3
    qt.k_scale = qt.v_scale = 1.0
    for k, v in kw.items():
        setattr(qt, k, v)
    return qt


def prefill_tile(head_dim, batch=0, n_heads=1, seq_len=0, causal=True):
    """Tile shape of the prefill kernel; with a batch of `batch` sequences of
    `seq_len` tokens over `n_heads` heads, kv_chunk = keys per KV chunk when
    the tile table splits such a call (0: no split)."""
    t = Ifa4Tile()
    a = make_args(head_dim=head_dim, batch=batch, n_heads=n_heads, kv_heads=1,
                  max_seqlen_q=seq_len, max_seqlen_k=seq_len, causal=int(causal))
    st = lib().ifa4_prefill_tile(ctypes.byref(a), ctypes.byref(t))
    if st != IFA4_OK:
        raise ValueError(status_str(st))
    return t


def count_tiles(cu_q, cu_k, n_heads, block_args=None, causal=True, window_left=-1,
                no_prune=False, head_dim=128, bottom_right=False):
    """KV tiles the prefill kernel visits vs an unpruned kernel (host count)."""
    batch = len(cu_q) - 1
    flags = (IFA4_FLAG_NO_PRUNE if no_prune else 0) | \
        (IFA4_FLAG_BOTTOM_RIGHT if bottom_right else 0)
    a = make_args(batch=batch, n_heads=n_heads, kv_heads=1, head_dim=head_dim,
                  causal=int(causal), window_left=window_left, flags=flags)
    cq = (ctypes.c_int32 * len(cu_q))(*[int(x) for x in cu_q])
    ck = (ctypes.c_int32 * len(cu_k))(*[int(x) for x in cu_k])
    vis, tot = ctypes.c_int64(), ctypes.c_int64()
    st = lib().ifa4_prefill_count_tiles(ctypes.byref(a), cq, ck, ctypes.byref(vis),
                                        ctypes.byref(tot))
    if st != IFA4_OK:
        raise ValueError(status_str(st))
    return vis.value, tot.value
