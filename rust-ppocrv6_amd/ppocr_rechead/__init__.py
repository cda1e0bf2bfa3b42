"""Host-side mirror of rust_ppocrv6's recognition-head operator API, on the MI355X library.

The names, argument meaning and error behaviour follow the reference's operators so a
caller (or a test) reads the same as against the Rust crate:

    QuantizedWeight.from_f32_transposed   src/ops/matmul.rs:1173-1202
    matmul_quantized_b                    src/ops/matmul.rs:1204-1336
    matmul_transposed_b                   src/ops/matmul.rs:514-897
    softmax / softmax_inplace             src/ops/softmax.rs:49-285
    CtcDecoder                            src/postprocess/ctc.rs:7-258
    RecHead.weight_footprint_bytes        src/engine/model.rs:651-667

Every computation runs in libppocr_rechead.so (hand-written gfx950 kernels).  Errors
come back as OcrError(op, msg), the shape of OcrError::OperatorError (src/error.rs).
"""
import ctypes
import os

import numpy as np

from . import _lib
from ._lib import (MODE_AUTO, MODE_BF16X1, MODE_BF16X2, MODE_BF16X3, MODE_F16X2, MODE_FP32_FMA, NECK_CHANNELS_FIRST,
                   NECK_ROWS, PPOCR_ERR_DEVICE, PPOCR_ERR_INVALID_ARG, PPOCR_ERR_MODEL, PPOCR_ERR_NO_MEMORY, PPOCR_OK)

__all__ = [
    "OcrError", "QuantizedWeight", "RecHead", "RecNeck", "CtcDecoder", "find_rec_head", "matmul_quantized_b", "matmul_transposed_b",
    "softmax", "softmax_inplace", "MODE_FP32_FMA", "MODE_BF16X1", "MODE_BF16X2", "MODE_BF16X3", "MODE_F16X2", "MODE_AUTO",
]


class OcrError(Exception):
    """OcrError::OperatorError { op, msg } (src/error.rs:4-27)."""

    def __init__(self, op, msg, code=PPOCR_ERR_INVALID_ARG):
        super().__init__(f"{op}: {msg}")
        self.op = op
        self.msg = msg
        self.code = code


def _check(rc):
    if rc != PPOCR_OK:
        text = _lib.last_error()
        op, _, msg = text.partition(": ")
        raise OcrError(op or "RecHeadHip", msg or text, rc)


def _ptr(arr):
    return None if arr is None else arr.ctypes.data_as(ctypes.c_void_p)


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


class QuantizedWeight:
    """Per-output-class symmetric INT8 weight (src/ops/matmul.rs:1165-1171).

    data: int8 [rows][cols], one row per output class; scales: f32 [rows]."""

    def __init__(self, data, scales):
        self.data = np.ascontiguousarray(data, dtype=np.int8)
        self.scales = np.ascontiguousarray(scales, dtype=np.float32)
        self.rows, self.cols = self.data.shape

    @classmethod
    def from_f32_transposed(cls, w_t):
        """Pack W^T [n][k] on the GPU, bit-exact with the reference packer."""
        w_t = _f32(w_t)
        if w_t.ndim != 2:
            raise OcrError("QuantizedWeight", f"expected a 2-D [n, k] weight, got shape {list(w_t.shape)}")
        n, k = w_t.shape
        q = np.empty((n, k), np.int8)
        s = np.empty(n, np.float32)
        if n:
            _check(_lib.lib().ppocr_rh_pack_int8(_ptr(w_t), n, k, _ptr(q), _ptr(s)))
        return cls(q, s)

    def nbytes(self):
        return self.data.size + 4 * self.scales.size


REC_HEAD_BACKENDS = ("cpu", "hip")


class OcrEngineConfig:
    """The recognition-head fields of OcrEngineConfig (src/pipeline.rs:38-40): the reference's
    INT8 switch `quantize_rec_head` (default False, bit-identical FP32 execution), unchanged,
    and where the head runs, `rec_head_backend`: "cpu" (the reference's own operators) or
    "hip" (this library on HIP device `rec_head_device`)."""

    def __init__(self, quantize_rec_head=False, rec_head_backend="cpu", rec_head_device=0):
        if rec_head_backend not in REC_HEAD_BACKENDS:
            raise OcrError("ModelError", f"unknown rec_head_backend {rec_head_backend!r} "
                                         f"(expected one of {', '.join(REC_HEAD_BACKENDS)})")
        self.quantize_rec_head = bool(quantize_rec_head)
        self.rec_head_backend = rec_head_backend
        self.rec_head_device = int(rec_head_device)

    def enable_rec_quantization(self):
        """OcrEngine::enable_rec_quantization (src/pipeline.rs:267-270): INT8 from now on; a
        head built for this configuration afterwards is the INT8 one."""
        self.quantize_rec_head = True


class RecHead:
    """The head weight resident in HBM: what Model keeps for MatMul.12 plus its folded bias.

    Build it once (INT8: from a QuantizedWeight; FP32: from W^T), then run any number of
    batches.  `mode` picks the arithmetic; the default, MODE_AUTO, takes the bf16 split
    (MODE_BF16X2 for INT8, MODE_BF16X3 for FP32) or MODE_F16X2, whichever the head's weights
    suit (auto_mode())."""

    def __init__(self, qw=None, bias=None, w_t=None, device=0):
        self._h = ctypes.c_void_p()
        bias_c = None if bias is None else _f32(bias)
        if qw is not None:
            if bias_c is not None and bias_c.size != qw.rows:
                raise OcrError("MatMulQuantized", f"bias has {bias_c.size} elements but n is {qw.rows}")
            self.quantized = True
            self.n, self.k = qw.rows, qw.cols
            _check(_lib.lib().ppocr_rh_create(_ptr(qw.data), _ptr(qw.scales), _ptr(bias_c), self.n, self.k, device,
                                              ctypes.byref(self._h)))
        else:
            w_t = _f32(w_t)
            if bias_c is not None and bias_c.size != w_t.shape[0]:
                raise OcrError("MatMulTransposedB", f"bias has {bias_c.size} elements but n is {w_t.shape[0]}")
            self.quantized = False
            self.n, self.k = w_t.shape
            _check(_lib.lib().ppocr_rh_create_f32(_ptr(w_t), _ptr(bias_c), self.n, self.k, device,
                                                  ctypes.byref(self._h)))
        self.default_mode = MODE_AUTO

    @classmethod
    def from_safetensors(cls, path, weight_name, bias_name=None, quantize=True, device=0):
        """The head straight from a model file (load_safetensors_model, src/engine/loader.rs:34-92,
        then the prepack and, with `quantize`, Model::quantize_matmul_weights): `weight_name`
        is the F32 [k][n] MatMul weight as stored, `bias_name` its F32 [n] bias.  Transpose,
        INT8 packing and the tile records run on the GPU."""
        self = cls.__new__(cls)
        self._h = ctypes.c_void_p()
        enc = (lambda x: None if x is None else os.fsencode(x))
        _check(_lib.lib().ppocr_rh_create_from_safetensors(enc(path), enc(weight_name), enc(bias_name),
                                                           1 if quantize else 0, device, ctypes.byref(self._h)))
        n, k, q = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int()
        _check(_lib.lib().ppocr_rh_shape(self._h, ctypes.byref(n), ctypes.byref(k), ctypes.byref(q)))
        self.n, self.k, self.quantized = n.value, k.value, bool(q.value)
        self.default_mode = MODE_AUTO
        return self

    @classmethod
    def from_model(cls, path, quantize=True, device=0):
        """The head of a model file, found in its graph (find_rec_head) and built on the
        GPU from the file's tensors (from_safetensors)."""
        names = find_rec_head(path)
        return cls.from_safetensors(path, names["weight"], names["bias"], quantize=quantize, device=device)

    @classmethod
    def for_config(cls, config, rec_path):
        """The head an engine with `config` uses for the recognition model at `rec_path`
        (OcrEngine::with_config, src/pipeline.rs:195-199): None for the "cpu" backend; for
        "hip", the INT8 head when quantize_rec_head is set (the packing of
        Model::quantize_matmul_weights) and the FP32 head otherwise."""
        if config.rec_head_backend == "cpu":
            return None
        return cls.from_model(rec_path, quantize=config.quantize_rec_head, device=config.rec_head_device)

    def close(self):
        if self._h:
            _lib.lib().ppocr_rh_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def weight_footprint_bytes(self):
        """This weight's share of Model::weight_footprint_bytes (src/engine/model.rs:651-667)."""
        return int(_lib.lib().ppocr_rh_footprint_bytes(self._h))

    def device_bytes(self):
        return int(_lib.lib().ppocr_rh_device_bytes(self._h))

    def auto_mode(self):
        """The mode MODE_AUTO (the default) runs for this head's weights."""
        return int(_lib.lib().ppocr_rh_auto_mode(self._h))

    def guard_limits(self, mode=None):
        """(prec, range_amax, range_norm): a row a takes the rescue pass of argmax / decode /
        probabilities when max|a| > prec or (max|a| > range_amax and ||a||_2 > range_norm),
        of logits when max|a| > prec (inf: no such limit in this mode)."""
        p, ra, rn = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
        _check(_lib.lib().ppocr_rh_guard_limits(self._h, self.default_mode if mode is None else mode,
                                                ctypes.byref(p), ctypes.byref(ra), ctypes.byref(rn)))
        return float(p.value), float(ra.value), float(rn.value)

    def guarded_rows(self, a, mode=None):
        """Which rows of a [rows][k] the statistics pass of `mode` sends to the rescue."""
        prec, ra, rn = self.guard_limits(mode)
        a = _f32(a).reshape(-1, self.k)
        amax = np.abs(a).max(axis=1) if a.size else np.zeros(0, np.float32)
        norm = np.sqrt((a.astype(np.float64) ** 2).sum(axis=1))
        return (amax > prec) | ((amax > ra) & (norm > rn))

    def workspace_bytes(self, m, mode=None):
        return int(_lib.lib().ppocr_rh_workspace_bytes(self._h, m, self.default_mode if mode is None else mode))

    def _rows(self, a, op):
        a = _f32(a)
        if a.ndim < 1:
            raise OcrError(op, "Operand must have valid dimensions")
        if a.shape[-1] != self.k:
            raise OcrError(op, f"Inner dimensions must match: {a.shape[-1]} != {self.k}")
        return a, a.size // self.k if self.k else 0

    def logits(self, a, mode=None):
        """MatMul.12: [.., m, k] -> [.., m, n] logits (matmul_quantized_b / matmul_transposed_b)."""
        op = "MatMulQuantizedB" if self.quantized else "MatMulTransposedB"
        a, rows = self._rows(a, op)
        out_shape = list(a.shape[:-1]) + [self.n] if a.ndim > 1 else [1, self.n]
        out = np.empty(out_shape, np.float32)
        if rows:
            _check(_lib.lib().ppocr_rh_logits(self._h, _ptr(a), rows, self.default_mode if mode is None else mode,
                                              _ptr(out)))
        return out

    def probs(self, a, mode=None):
        """MatMul.12 -> Softmax.2 in one call: [.., m, k] -> [.., m, n] probabilities."""
        a, rows = self._rows(a, "RecHeadHip")
        out = np.empty(list(a.shape[:-1]) + [self.n], np.float32)
        if rows:
            _check(_lib.lib().ppocr_rh_probs(self._h, _ptr(a), rows, self.default_mode if mode is None else mode,
                                             _ptr(out)))
        return out

    def argmax(self, a, mode=None):
        """Per row: first-index argmax of the softmax and the max probability."""
        a, rows = self._rows(a, "RecHeadHip")
        idx = np.empty(rows, np.int32)
        mp = np.empty(rows, np.float32)
        if rows:
            _check(_lib.lib().ppocr_rh_argmax(self._h, _ptr(a), rows, self.default_mode if mode is None else mode,
                                              _ptr(idx), _ptr(mp)))
        return idx, mp

    def decode(self, a, line_off, mode=None):
        """Whole head over text lines packed back to back: index sequences and scores."""
        a = _f32(a).reshape(-1, self.k) if self.k else _f32(a)
        line_off = np.ascontiguousarray(line_off, dtype=np.int64)
        lines = line_off.size - 1
        m = int(line_off[-1]) if lines >= 0 else 0
        if lines < 0:
            raise OcrError("CtcDecode", "line offsets must hold at least one entry")
        if m != a.shape[0]:
            raise OcrError("CtcDecode", f"line offsets cover {m} rows but the input has {a.shape[0]}")
        idx = np.empty(max(m, 1), np.int32)
        mp = np.empty(max(m, 1), np.float32)
        seq = np.zeros(max(m, 1), np.int32)
        seq_len = np.zeros(max(lines, 1), np.int64)
        score = np.zeros(max(lines, 1), np.float32)
        if lines:
            _check(_lib.lib().ppocr_rh_decode(self._h, _ptr(a), _ptr(line_off), lines,
                                              self.default_mode if mode is None else mode, _ptr(idx), _ptr(mp),
                                              _ptr(seq), _ptr(seq_len), _ptr(score)))
        seqs = [seq[line_off[b]:line_off[b] + seq_len[b]].copy() for b in range(lines)]
        return {"idx": idx[:m], "maxprob": mp[:m], "seqs": seqs, "score": score[:lines]}

    def decode_nct(self, x, mode=None):
        """Whole head from the neck's output before its transpose (Transpose.8, perm
        [0,2,1]; src/engine/model.rs:1325-1342): x [lines, k, T], channels first.  The
        same results as decode() on x.transpose(0, 2, 1) with T steps per line."""
        x = _f32(x)
        if x.ndim != 3 or x.shape[1] != self.k:
            raise OcrError("RecHeadHip", f"expected [lines, {self.k}, T], got {list(x.shape)}")
        lines, _, steps = x.shape
        m = lines * steps
        idx = np.empty(max(m, 1), np.int32)
        mp = np.empty(max(m, 1), np.float32)
        seq = np.zeros(max(m, 1), np.int32)
        seq_len = np.zeros(max(lines, 1), np.int64)
        score = np.zeros(max(lines, 1), np.float32)
        if lines:
            _check(_lib.lib().ppocr_rh_decode_nct(self._h, _ptr(x), lines, steps,
                                                  self.default_mode if mode is None else mode, _ptr(idx), _ptr(mp),
                                                  _ptr(seq), _ptr(seq_len), _ptr(score)))
        seqs = [seq[b * steps:b * steps + seq_len[b]].copy() for b in range(lines)]
        return {"idx": idx[:m], "maxprob": mp[:m], "seqs": seqs, "score": score[:lines]}


class RecNeck:
    """The recognition model's SVTR mixing tail before the head, resident in HBM: the
    transformer blocks, final LayerNorm and shortcut Add between Transpose.0 and
    Transpose.8 of PP-OCRv6_small_rec, which the reference's executor runs node by node
    (Model::forward, src/engine/model.rs: MatMul 1245-1272, LayerNorm 1274-1284, Softmax
    1286-1302, Sigmoid 953-963).

    blocks: list of dicts with the fields of ppocr_rn_block_t (ln1_w, ln1_b, ln1_eps,
    qkv_w [D][3D], qkv_b, proj_w [D][D], proj_b, ln2_w, ln2_b, ln2_eps, fc1_w [D][H], fc1_b,
    fc2_w [H][D], fc2_b), MatMul weights row-major [K][N] as the model stores them."""

    _FIELDS = ("ln1_w", "ln1_b", "qkv_w", "qkv_b", "proj_w", "proj_b", "ln2_w", "ln2_b", "fc1_w", "fc1_b",
               "fc2_w", "fc2_b")

    def __init__(self, blocks, lnf_w, lnf_b, lnf_eps, heads=8, scale=None, device=0):
        self._h = ctypes.c_void_p()
        keep = []

        def arr(x):
            a = _f32(x)
            keep.append(a)
            return a.ctypes.data_as(ctypes.c_void_p)

        dim = int(np.asarray(blocks[0]["ln1_w"]).size)
        hidden = int(np.asarray(blocks[0]["fc1_b"]).size)
        if scale is None:
            scale = float(np.float32((dim // heads) ** -0.5))
        cb = (_lib.RnBlock * len(blocks))()
        for i, b in enumerate(blocks):
            for f in self._FIELDS:
                setattr(cb[i], f, arr(b[f]))
            cb[i].ln1_eps = float(b["ln1_eps"])
            cb[i].ln2_eps = float(b["ln2_eps"])
        _check(_lib.lib().ppocr_rn_create(cb, len(blocks), arr(lnf_w), arr(lnf_b), float(lnf_eps), dim, heads, hidden,
                                          float(scale), device, ctypes.byref(self._h)))
        self.dim, self.heads, self.hidden, self.blocks = dim, heads, hidden, len(blocks)

    @classmethod
    def from_model(cls, path, device=0):
        """The tail of a recognition model file (its graph searched from the first
        LayerNorm to the head's MatMul), weights uploaded from the file."""
        self = cls.__new__(cls)
        self._h = ctypes.c_void_p()
        _check(_lib.lib().ppocr_rn_create_from_model(os.fsencode(path), device, ctypes.byref(self._h)))
        d, h, f, b = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int()
        _check(_lib.lib().ppocr_rn_shape(self._h, ctypes.byref(d), ctypes.byref(h), ctypes.byref(f), ctypes.byref(b)))
        self.dim, self.heads, self.hidden, self.blocks = d.value, h.value, f.value, b.value
        return self

    def close(self):
        if self._h:
            _lib.lib().ppocr_rn_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    @property
    def gemm_halves(self):
        """True when the tail's MatMuls run on fp16 halves of both operands (three exact
        products summed in fp32), False on fp32 products."""
        r = _lib.lib().ppocr_rn_gemm_halves(self._h)
        if r < 0:
            _check(r)
        return r == 1

    def workspace_bytes(self, m):
        return int(_lib.lib().ppocr_rn_workspace_bytes(self._h, m))

    def forward(self, x, shortcut, line_off, layout=_lib.NECK_ROWS):
        """Token rows [m][D] (the head's input) from x and shortcut in `layout`: token rows
        [m][D], or channels first (line b as [D][T_b] at D * line_off[b])."""
        line_off = np.ascontiguousarray(line_off, dtype=np.int64)
        lines = line_off.size - 1
        if lines < 0:
            raise OcrError("RecNeckHip", "line offsets must hold at least one entry")
        m = int(line_off[-1])
        x = _f32(x).reshape(-1)
        shortcut = _f32(shortcut).reshape(-1)
        if x.size != m * self.dim or shortcut.size != m * self.dim:
            raise OcrError("RecNeckHip", f"expected {m} x {self.dim} values in x and shortcut")
        out = np.empty((m, self.dim), np.float32)
        if m:
            _check(_lib.lib().ppocr_rn_forward(self._h, _ptr(x), _ptr(shortcut), _ptr(line_off), lines, layout,
                                               _ptr(out)))
        return out


def find_rec_head(path):
    """The recognition head of a model file: the MatMul -> [Add bias] -> Softmax(last axis) ->
    graph output segment of its graph, as {"weight", "bias" (None if absent), "n", "k"}
    (the segment the engine-level fused hook replaces)."""
    wb, bb = ctypes.create_string_buffer(1024), ctypes.create_string_buffer(1024)
    n, k = ctypes.c_int64(), ctypes.c_int64()
    _check(_lib.lib().ppocr_model_find_rec_head(os.fsencode(path), wb, 1024, bb, 1024, ctypes.byref(n),
                                                ctypes.byref(k)))
    bias = os.fsdecode(bb.value)
    return {"weight": os.fsdecode(wb.value), "bias": bias or None, "n": n.value, "k": k.value}


def matmul_quantized_b(a, qw, bias=None, mode=MODE_AUTO):
    """matmul_quantized_b(a, qw, bias) (src/ops/matmul.rs:1204-1336) on the GPU, in the
    library's default arithmetic unless `mode` says otherwise.  The head (the packed weight
    and its tile records in HBM) is built on the first call with a given QuantizedWeight and
    bias and kept on that QuantizedWeight, as Model keeps its packed weight resident; a
    QuantizedWeight is not modified after it is built (the reference's is immutable)."""
    a = _f32(a)
    if a.ndim < 1:
        raise OcrError("MatMulQuantizedB", "Operand must have valid dimensions")
    if a.shape[-1] != qw.cols:
        raise OcrError("MatMulQuantizedB", f"Inner dimensions must match: {a.shape[-1]} != {qw.cols}")
    if bias is not None and np.asarray(bias).size != qw.rows:
        raise OcrError("MatMulQuantized", f"bias has {np.asarray(bias).size} elements but n is {qw.rows}")
    b = None if bias is None else _f32(bias)
    key = None if b is None else b.tobytes()
    heads = qw.__dict__.setdefault("_gpu_heads", {})
    head = heads.get(key)
    if head is None:
        head = heads[key] = RecHead(qw=qw, bias=b)
    return head.logits(a, mode)


def matmul_transposed_b(a, b_t, bias=None, mode=MODE_AUTO):
    """matmul_transposed_b(a, b_t, bias) (src/ops/matmul.rs:514-897) on the GPU, in the
    library's default arithmetic unless `mode` says otherwise.  The FP32 head is built for
    the call (b_t is a plain array that may change between calls); for repeated calls with
    one weight build a RecHead(w_t=...) once, as Model keeps its transposed weight."""
    a = _f32(a)
    b_t = _f32(b_t)
    if a.ndim < 1 or b_t.ndim != 2:
        raise OcrError("MatMulTransposedB", "Operands must have valid dimensions")
    if a.shape[-1] != b_t.shape[1]:
        raise OcrError("MatMulTransposedB", f"Inner dimensions must match: {a.shape[-1]} != {b_t.shape[1]}")
    if bias is not None and np.asarray(bias).size != b_t.shape[0]:
        raise OcrError("MatMulTransposedB", f"bias has {np.asarray(bias).size} elements but n is {b_t.shape[0]}")
    head = RecHead(w_t=b_t, bias=bias)
    try:
        return head.logits(a, mode)
    finally:
        head.close()


def _norm_axis(ndim, axis):
    ax = axis + ndim if axis < 0 else axis
    if ax < 0 or ax >= ndim:
        raise OcrError("Softmax", f"Axis {axis} out of bounds for ndim {ndim}")
    return ax


def softmax_inplace(x, axis=-1):
    """softmax_inplace(x, axis) (src/ops/softmax.rs:199-285) over the last axis, on the GPU."""
    if not isinstance(x, np.ndarray) or x.dtype != np.float32 or not x.flags.c_contiguous:
        raise OcrError("Softmax", "softmax_inplace needs a C-contiguous float32 numpy array")
    ax = _norm_axis(x.ndim, axis)
    if ax != x.ndim - 1:
        raise OcrError("Softmax", "only the last axis (the classifier axis) is offloaded")
    if x.size == 0:
        return
    cols = x.shape[-1]
    _check(_lib.lib().ppocr_softmax_rows(_ptr(x), x.size // cols, cols))


def softmax(x, axis=-1):
    """softmax(x, axis) (src/ops/softmax.rs:49-197): a new array."""
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    _norm_axis(x.ndim, axis)
    softmax_inplace(x, axis)
    return x


class CtcDecoder:
    """CTC greedy decoder (src/postprocess/ctc.rs:7-175); argmax and collapse on the GPU."""

    def __init__(self, vocab):
        self.vocab = list(vocab)

    @classmethod
    def from_file(cls, dict_path):
        """vocab = ["blank"] + dictionary lines + [" "] (src/postprocess/ctc.rs:12-30).

        Lines as BufRead::lines gives them: split on '\n' only (a '\r' inside a line stays
        in it), no empty line after a final '\n', then trailing '\r' and '\n' trimmed.
        Text that is not UTF-8 is a ModelError ("Dict read error")."""
        try:
            with open(dict_path, "rb") as f:
                data = f.read()
        except OSError as e:
            raise OcrError("ModelError", f"Failed to open dict file: {e}")
        try:
            text = data.decode("utf-8")
        except UnicodeDecodeError as e:
            raise OcrError("ModelError", f"Dict read error: {e}")
        lines = text.split("\n")
        if lines and lines[-1] == "":
            lines = lines[:-1]
        vocab = ["blank"] + [ln.rstrip("\r\n") for ln in lines] + [" "]
        return cls(vocab)

    @classmethod
    def from_vocab(cls, vocab):
        return cls(vocab)

    def vocab_size(self):
        return len(self.vocab)

    def _check_preds(self, preds):
        preds = np.asarray(preds)
        if preds.ndim != 3:
            raise OcrError("CtcDecode", f"Expected 3D tensor [batch, time, vocab], got shape {list(preds.shape)}")
        if preds.shape[2] != len(self.vocab):
            raise OcrError("CtcDecode", f"dictionary/model mismatch: model outputs {preds.shape[2]} classes but the "
                                        f"dictionary has {len(self.vocab)} entries")
        return _f32(preds)

    def decode(self, preds):
        """First line of decode_batch; ("", 0.0) for an empty batch (src/postprocess/ctc.rs:40-100)."""
        preds = self._check_preds(preds)
        if preds.shape[0] == 0 or preds.shape[1] == 0:
            return "", 0.0
        return self.decode_batch(preds)[0]

    def decode_batch(self, preds):
        """[batch, time, vocab] probabilities -> [(text, score)] (src/postprocess/ctc.rs:103-175)."""
        preds = self._check_preds(preds)
        b, t, c = preds.shape
        if b == 0 or t == 0:
            return []
        rows = b * t
        idx = np.empty(rows, np.int32)
        val = np.empty(rows, np.float32)
        _check(_lib.lib().ppocr_argmax_rows(_ptr(preds), rows, c, _ptr(idx), _ptr(val)))
        line_off = np.arange(0, rows + 1, t, dtype=np.int64)
        return self.decode_steps(idx, val, line_off)

    def decode_steps(self, idx, maxprob, line_off):
        """Collapse per-step (argmax, max probability) of lines given by offsets into text."""
        seqs, scores = self.collapse(idx, maxprob, line_off)
        return [("".join(self.vocab[j] for j in s), float(sc)) for s, sc in zip(seqs, scores)]

    @staticmethod
    def collapse(idx, maxprob, line_off, blank=0):
        idx = np.ascontiguousarray(idx, dtype=np.int32)
        maxprob = _f32(maxprob)
        line_off = np.ascontiguousarray(line_off, dtype=np.int64)
        lines = line_off.size - 1
        seq = np.zeros(max(idx.size, 1), np.int32)
        seq_len = np.zeros(max(lines, 1), np.int64)
        score = np.zeros(max(lines, 1), np.float32)
        if lines > 0:
            _check(_lib.lib().ppocr_ctc_greedy(_ptr(idx), _ptr(maxprob), _ptr(line_off), lines, blank, _ptr(seq),
                                               _ptr(seq_len), _ptr(score)))
        return [seq[line_off[b]:line_off[b] + seq_len[b]].copy() for b in range(lines)], score[:max(lines, 0)].copy()
