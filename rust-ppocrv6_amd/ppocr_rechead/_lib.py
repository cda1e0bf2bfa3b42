"""ctypes binding of libppocr_rechead.so (the C ABI in include/ppocr_rechead.h).

The library is the product: every compute entry point runs hand-written HIP kernels on
the GPU.  There is no CPU fallback; if the library is missing, loading fails loudly.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("PPOCR_RECHEAD_LIB",
                          os.path.normpath(os.path.join(_HERE, "..", "lib", "libppocr_rechead.so")))

PPOCR_OK = 0
PPOCR_ERR_INVALID_ARG = 1
PPOCR_ERR_DEVICE = 2
PPOCR_ERR_NO_MEMORY = 3
PPOCR_ERR_MODEL = 4

MODE_FP32_FMA = 0
MODE_BF16X1 = 1
MODE_BF16X2 = 2
MODE_BF16X3 = 3
MODE_F16X2 = 4
MODE_AUTO = 5

NECK_ROWS = 0
NECK_CHANNELS_FIRST = 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_int = ctypes.c_int
_sz = ctypes.c_size_t



class RnBlock(ctypes.Structure):
    """ppocr_rn_block_t: one transformer block's weights (host pointers)."""
    _fields_ = [("ln1_w", _vp), ("ln1_b", _vp), ("ln1_eps", ctypes.c_float), ("qkv_w", _vp), ("qkv_b", _vp),
                ("proj_w", _vp), ("proj_b", _vp), ("ln2_w", _vp), ("ln2_b", _vp), ("ln2_eps", ctypes.c_float),
                ("fc1_w", _vp), ("fc1_b", _vp), ("fc2_w", _vp), ("fc2_b", _vp)]


# name -> (restype, argtypes); every function declared in include/ppocr_rechead.h.
SIGNATURES = {
    "ppocr_last_error": (ctypes.c_char_p, []),
    "ppocr_rh_pack_int8": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "ppocr_rh_pack_int8_dev": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "ppocr_rh_create": (_int, [_vp, _vp, _vp, _i64, _i64, _int, ctypes.POINTER(_vp)]),
    "ppocr_rh_create_f32": (_int, [_vp, _vp, _i64, _i64, _int, ctypes.POINTER(_vp)]),
    "ppocr_rh_create_from_safetensors": (_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _int, _int,
                                                ctypes.POINTER(_vp)]),
    "ppocr_model_find_rec_head": (_int, [ctypes.c_char_p, ctypes.c_char_p, _sz, ctypes.c_char_p, _sz,
                                         ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "ppocr_rh_destroy": (None, [_vp]),
    "ppocr_rh_footprint_bytes": (_sz, [_vp]),
    "ppocr_rh_device_bytes": (_sz, [_vp]),
    "ppocr_rh_shape": (_int, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_int)]),
    "ppocr_rh_auto_mode": (_int, [_vp]),
    "ppocr_rh_guard_limits": (_int, [_vp, _int, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float),
                                     ctypes.POINTER(ctypes.c_float)]),
    "ppocr_rh_workspace_bytes": (_sz, [_vp, _i64, _int]),
    "ppocr_rh_logits": (_int, [_vp, _vp, _i64, _int, _vp]),
    "ppocr_rh_logits_dev": (_int, [_vp, _vp, _i64, _int, _vp, _vp, _sz, _vp]),
    "ppocr_softmax_rows": (_int, [_vp, _i64, _i64]),
    "ppocr_softmax_rows_dev": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "ppocr_argmax_rows": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "ppocr_argmax_rows_dev": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "ppocr_rh_probs": (_int, [_vp, _vp, _i64, _int, _vp]),
    "ppocr_rh_probs_dev": (_int, [_vp, _vp, _i64, _int, _vp, _vp, _sz, _vp]),
    "ppocr_rh_argmax": (_int, [_vp, _vp, _i64, _int, _vp, _vp]),
    "ppocr_rh_argmax_dev": (_int, [_vp, _vp, _i64, _int, _vp, _vp, _vp, _sz, _vp]),
    "ppocr_ctc_greedy": (_int, [_vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp]),
    "ppocr_ctc_greedy_dev": (_int, [_vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp]),
    "ppocr_rh_decode": (_int, [_vp, _vp, _vp, _i64, _int, _vp, _vp, _vp, _vp, _vp]),
    "ppocr_rh_decode_dev": (_int, [_vp, _vp, _i64, _vp, _i64, _int, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ppocr_rh_decode_dev_noalloc": (_int, [_vp, _vp, _i64, _vp, _i64, _int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ppocr_rh_decode_nct": (_int, [_vp, _vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _vp]),
    "ppocr_rh_decode_nct_dev": (_int, [_vp, _vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ppocr_rn_create": (_int, [ctypes.POINTER(RnBlock), _int, _vp, _vp, ctypes.c_float, _i64, _i64, _i64,
                               ctypes.c_float, _int, ctypes.POINTER(_vp)]),
    "ppocr_rn_create_from_model": (_int, [ctypes.c_char_p, _int, ctypes.POINTER(_vp)]),
    "ppocr_rn_destroy": (None, [_vp]),
    "ppocr_rn_shape": (_int, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                              ctypes.POINTER(_int)]),
    "ppocr_rn_gemm_halves": (_int, [_vp]),
    "ppocr_rn_workspace_bytes": (_sz, [_vp, _i64]),
    "ppocr_rn_forward_dev": (_int, [_vp, _vp, _vp, _i64, _vp, _i64, _int, _vp, _vp, _sz, _vp]),
    "ppocr_rn_forward": (_int, [_vp, _vp, _vp, _vp, _i64, _int, _vp]),
    "ppocr_rn_forward_marked_dev": (_int, [_vp, _vp, _vp, _i64, _vp, _i64, _int, _vp, _vp, _sz, _vp,
                                           ctypes.POINTER(_vp), _int, ctypes.POINTER(ctypes.c_char_p),
                                           ctypes.POINTER(_int)]),
}

_lib = None


def lib():
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libppocr_rechead.so not found at {LIB_PATH}; build it with "
                               "`make -C rust-ppocrv6_amd/csrc` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    msg = lib().ppocr_last_error()
    return msg.decode() if msg else ""
