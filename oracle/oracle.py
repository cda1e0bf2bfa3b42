"""ctypes front end of the CPU oracle (oracle/rechead_oracle.c).

TEST INFRASTRUCTURE ONLY.  The oracle restates the reference's CPU path for the
recognition head (packer, W8A32 projection, FP32 projection, softmax, argmax, CTC
collapse) with the reference's own AVX2 intrinsic sequence, and the SVTR neck tail before
it (LayerNorm, sigmoid, the activation MatMuls, attention) from the same pieces.  Only tests/, the smoke
check in __graft_entry__.py and the CPU-baseline leg of bench.py import this module;
the product package never does.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle_rechead.so")

_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int


def lib():
    """Load the oracle library (built by `make -C oracle`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_pack_int8.argtypes = [_f32p, _i64, _i64, _i8p, _f32p]
        L.orc_pack_int8.restype = None
        L.orc_matmul_quantized_b.argtypes = [_f32p, _i64, _i8p, _f32p, ctypes.c_void_p, _i64, _i64,
                                             _int, _int, _int, _f32p]
        L.orc_matmul_quantized_b.restype = None
        L.orc_matmul_transposed_b.argtypes = [_f32p, _i64, _f32p, ctypes.c_void_p, _i64, _i64,
                                              _int, _int, _int, _f32p]
        L.orc_matmul_transposed_b.restype = None
        L.orc_exp_ps.argtypes = [_f32p, _i64, _f32p]
        L.orc_exp_ps.restype = None
        L.orc_softmax_rows.argtypes = [_f32p, _i64, _i64, _int, _int]
        L.orc_softmax_rows.restype = None
        L.orc_find_argmax.argtypes = [_f32p, _i64, _int, ctypes.POINTER(ctypes.c_float)]
        L.orc_find_argmax.restype = _i64
        L.orc_argmax_rows.argtypes = [_f32p, _i64, _i64, _int, _int, _i32p, _f32p]
        L.orc_argmax_rows.restype = None
        L.orc_ctc_collapse.argtypes = [_i32p, _f32p, _i64p, _i64, ctypes.c_int32, _i32p, _i64p, _f32p]
        L.orc_ctc_collapse.restype = None
        L.orc_rechead_lines.argtypes = [_f32p, _i64p, _i64, _i8p, _f32p, ctypes.c_void_p, _i64, _i64,
                                        _int, _int, _i32p, _f32p, _i32p, _i64p, _f32p, ctypes.c_void_p]
        L.orc_rechead_lines.restype = None
        L.orc_layer_norm_rows.argtypes = [_f32p, _i64, _i64, _f32p, _f32p, ctypes.c_float, _int, _f32p]
        L.orc_layer_norm_rows.restype = None
        L.orc_sigmoid.argtypes = [_f32p, _i64, _f32p]
        L.orc_sigmoid.restype = None
        _lib = L
    return _lib


def _c(x, dt):
    return np.ascontiguousarray(x, dtype=dt)


def _opt_ptr(x):
    return None if x is None else x.ctypes.data_as(ctypes.c_void_p)


def default_threads():
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def pack_int8(w_t):
    """QuantizedWeight::from_f32_transposed (src/ops/matmul.rs:1173-1202)."""
    w_t = _c(w_t, np.float32)
    n, k = w_t.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    lib().orc_pack_int8(w_t, n, k, q, s)
    return q, s


def matmul_quantized_b(a, q, scales, bias=None, partition_threads=1, use_avx2=True, exec_threads=None):
    """matmul_quantized_b (src/ops/matmul.rs:1204-1336) over a [rows, k]."""
    a = _c(a, np.float32)
    q = _c(q, np.int8)
    scales = _c(scales, np.float32)
    n, k = q.shape
    rows = a.size // k
    bias_c = None if bias is None else _c(bias, np.float32)
    out = np.empty((rows, n), np.float32)
    lib().orc_matmul_quantized_b(a.reshape(-1), rows, q, scales, _opt_ptr(bias_c), n, k,
                                 int(partition_threads), int(bool(use_avx2)),
                                 int(exec_threads or default_threads()), out)
    return out


def matmul_transposed_b(a, w_t, bias=None, partition_threads=1, use_avx2=True, exec_threads=None):
    """matmul_transposed_b (src/ops/matmul.rs:514-897) over a [rows, k]."""
    a = _c(a, np.float32)
    w_t = _c(w_t, np.float32)
    n, k = w_t.shape
    rows = a.size // k
    bias_c = None if bias is None else _c(bias, np.float32)
    out = np.empty((rows, n), np.float32)
    lib().orc_matmul_transposed_b(a.reshape(-1), rows, w_t, _opt_ptr(bias_c), n, k,
                                  int(partition_threads), int(bool(use_avx2)),
                                  int(exec_threads or default_threads()), out)
    return out


def exp_ps(x):
    """avx2_exp_ps (src/ops/softmax.rs:5-47) elementwise; len(x) % 8 == 0."""
    x = _c(x, np.float32).reshape(-1)
    assert x.size % 8 == 0
    out = np.empty_like(x)
    lib().orc_exp_ps(x, x.size, out)
    return out


def softmax_rows(x, use_avx2=True, exec_threads=None):
    """softmax_inplace over the last axis (src/ops/softmax.rs:199-285); returns a copy."""
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    n = x.shape[-1] if x.ndim else 1
    rows = x.size // n if n else 0
    if x.size:
        lib().orc_softmax_rows(x.reshape(-1), rows, n, int(bool(use_avx2)),
                               int(exec_threads or default_threads()))
    return x


def find_argmax(x, use_avx2=True):
    """find_argmax (src/postprocess/ctc.rs:178-258) -> (index, value)."""
    x = _c(x, np.float32).reshape(-1)
    v = ctypes.c_float()
    if x.size == 0:
        x = np.zeros(1, np.float32)
        i = lib().orc_find_argmax(x, 0, int(bool(use_avx2)), ctypes.byref(v))
    else:
        i = lib().orc_find_argmax(x, x.size, int(bool(use_avx2)), ctypes.byref(v))
    return int(i), float(v.value)


def argmax_rows(probs, use_avx2=True, exec_threads=None):
    probs = _c(probs, np.float32)
    n = probs.shape[-1]
    rows = probs.size // n
    idx = np.empty(rows, np.int32)
    val = np.empty(rows, np.float32)
    lib().orc_argmax_rows(probs.reshape(-1), rows, n, int(bool(use_avx2)),
                          int(exec_threads or default_threads()), idx, val)
    return idx, val


def ctc_collapse(idx, val, line_off, blank=0):
    """decode_batch collapse/score (src/postprocess/ctc.rs:144-172) from per-step argmax."""
    idx = _c(idx, np.int32)
    val = _c(val, np.float32)
    line_off = _c(line_off, np.int64)
    lines = line_off.size - 1
    seq = np.zeros(max(idx.size, 1), np.int32)
    seq_len = np.zeros(max(lines, 1), np.int64)
    score = np.zeros(max(lines, 1), np.float32)
    if lines > 0:
        lib().orc_ctc_collapse(idx if idx.size else np.zeros(1, np.int32),
                               val if val.size else np.zeros(1, np.float32),
                               line_off, lines, blank, seq, seq_len, score)
    return [seq[line_off[b]:line_off[b] + seq_len[b]].copy() for b in range(lines)], score[:lines].copy()


def rechead_lines(a, line_off, q, scales, bias, use_avx2=True, exec_threads=None, want_probs=False):
    """Whole head per text line, one line per worker (src/pipeline.rs:417-433)."""
    a = _c(a, np.float32)
    q = _c(q, np.int8)
    scales = _c(scales, np.float32)
    line_off = _c(line_off, np.int64)
    n, k = q.shape
    rows = a.size // k
    lines = line_off.size - 1
    bias_c = None if bias is None else _c(bias, np.float32)
    idx = np.empty(max(rows, 1), np.int32)
    maxprob = np.empty(max(rows, 1), np.float32)
    seq = np.zeros(max(rows, 1), np.int32)
    seq_len = np.zeros(max(lines, 1), np.int64)
    score = np.zeros(max(lines, 1), np.float32)
    probs = np.empty((rows, n), np.float32) if want_probs else None
    lib().orc_rechead_lines(a.reshape(-1) if a.size else np.zeros(1, np.float32), line_off, lines, q, scales,
                            _opt_ptr(bias_c), n, k, int(bool(use_avx2)),
                            int(exec_threads or default_threads()), idx, maxprob, seq, seq_len, score,
                            _opt_ptr(probs))
    seqs = [seq[line_off[b]:line_off[b] + seq_len[b]].copy() for b in range(lines)]
    return {"idx": idx[:rows], "maxprob": maxprob[:rows], "seqs": seqs, "score": score[:lines],
            "probs": probs}


# ---------------------------------------------------------------- the SVTR neck tail
def layer_norm_rows(x, w, b, eps, use_avx2=True):
    """layer_norm over the last axis (src/ops/layernorm.rs:5-244)."""
    x = _c(x, np.float32)
    n = x.shape[-1]
    out = np.empty_like(x)
    if x.size:
        lib().orc_layer_norm_rows(x.reshape(-1), x.size // n, n, _c(w, np.float32), _c(b, np.float32),
                                  float(eps), int(bool(use_avx2)), out.reshape(-1))
    return out


def sigmoid(x):
    """sigmoid_inplace (src/ops/activation.rs:31-94) on a copy."""
    x = _c(x, np.float32)
    out = np.empty_like(x)
    if x.size:
        lib().orc_sigmoid(x.reshape(-1), x.size, out.reshape(-1))
    return out


def matmul_act(a, w):
    """MatMul of an activation by a weight or another activation (matmul_with_bias without
    bias, src/ops/matmul.rs:9-96, whose parallel_sgemm_2d / gemm_row_major blocking is not
    restated): the products summed in float64 and rounded once to float32, the correctly
    rounded value every fp32 summation order approximates."""
    return (np.asarray(a, np.float64) @ np.asarray(w, np.float64)).astype(np.float32)


def linear(a, w, bias):
    """MatMul then Add(bias), two nodes and two roundings (src/engine/model.rs:1245-1272)."""
    return (matmul_act(a, w) + _c(bias, np.float32)).astype(np.float32)


def attention_line(qkv, heads, scale):
    """The attention of one line's T tokens (graph nodes Reshape [0,-1,3,H,D/H], Transpose
    [2,0,3,1,4], Mul(scale), MatMul(q, k^T), Softmax over the keys (softmax_inplace,
    src/ops/softmax.rs:199-285), MatMul(p, v), Transpose [0,2,1,3], Reshape [0,-1,D]):
    qkv [T][3D] -> [T][D]."""
    t, d3 = qkv.shape
    d = d3 // 3
    hd = d // heads
    x = qkv.reshape(t, 3, heads, hd).transpose(1, 2, 0, 3)  # [3][H][T][hd]
    out = np.empty((heads, t, hd), np.float32)
    for h in range(heads):
        q = (x[0, h] * np.float32(scale)).astype(np.float32)
        s = matmul_act(q, x[1, h].T)
        p = softmax_rows(s)
        out[h] = matmul_act(p, x[2, h])
    return out.transpose(1, 0, 2).reshape(t, d)


def svtr_neck(x, shortcut, line_off, blocks, lnf_w, lnf_b, lnf_eps, heads, scale):
    """The SVTR tail on token rows x [m][D] (after Transpose.0), lines by line_off, blocks a
    list of dicts with the fields of ppocr_rn_block_t: per block
    x = x + proj(attention(LN1(x))), x = x + fc2(swish(fc1(LN2(x)))) (swish = Mul(h,
    Sigmoid(h))); then LN(x) + shortcut (rows [m][D])."""
    x = _c(x, np.float32).copy()
    line_off = np.asarray(line_off, np.int64)
    for b in blocks:
        y = layer_norm_rows(x, b["ln1_w"], b["ln1_b"], b["ln1_eps"])
        qkv = linear(y, b["qkv_w"], b["qkv_b"])
        att = np.zeros_like(x)
        for i in range(line_off.size - 1):
            t0, t1 = int(line_off[i]), int(line_off[i + 1])
            if t1 > t0:
                att[t0:t1] = attention_line(qkv[t0:t1], heads, scale)
        x = (x + linear(att, b["proj_w"], b["proj_b"])).astype(np.float32)
        y = layer_norm_rows(x, b["ln2_w"], b["ln2_b"], b["ln2_eps"])
        h = linear(y, b["fc1_w"], b["fc1_b"])
        h = (h * sigmoid(h)).astype(np.float32)
        x = (x + linear(h, b["fc2_w"], b["fc2_b"])).astype(np.float32)
    return (layer_norm_rows(x, lnf_w, lnf_b, lnf_eps) + _c(shortcut, np.float32)).astype(np.float32)
