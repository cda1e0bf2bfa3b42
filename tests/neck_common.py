"""Helpers of the SVTR neck tests: seeded synthetic weights with the statistics of
PP-OCRv6_small_rec's tail, a model file holding such a tail in its graph, and a small
interpreter of the graph's nodes with ONNX semantics (used to pin the oracle's wiring
against the graph itself)."""
import json
import struct

import numpy as np

DIM, HEADS, HIDDEN = 120, 8, 240
SCALE = np.float32(15 ** -0.5)


def neck_weights(seed=7, blocks=2):
    """Seeded synthetic tail weights (ppocr_rechead.workloads.neck_weights)."""
    from ppocr_rechead import workloads as wl
    return wl.neck_weights(seed=seed, blocks=blocks)


def lines_of(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)


def rows_to_cf(rows, line_off):
    """Token rows [m][D] to channels-first lines (line b as [D][T_b] at D * line_off[b])."""
    out = np.empty(rows.size, np.float32)
    d = rows.shape[1]
    for b in range(line_off.size - 1):
        t0, t1 = int(line_off[b]), int(line_off[b + 1])
        out[d * t0:d * t1] = rows[t0:t1].T.reshape(-1)
    return out


def oracle_neck(orc, w, x, shortcut, line_off):
    return orc.svtr_neck(x, shortcut, line_off, w["blocks"], w["lnf_w"], w["lnf_b"], w["lnf_eps"], HEADS, SCALE)


# ---------------------------------------------------------------- a model file with the tail
class _G:
    def __init__(self):
        self.nodes, self.tensors, self.n = [], {}, 0

    def const(self, name, arr):
        self.tensors[name] = np.ascontiguousarray(arr)
        return name

    def node(self, op, inputs, attrs=None, n_out=1):
        self.n += 1
        outs = [f"v{self.n}_{k}" for k in range(n_out)]
        self.nodes.append({"name": f"{op}.{self.n}", "op": op, "inputs": list(inputs), "outputs": outs,
                           "attrs": attrs or {}})
        return outs[0]


def _layer_norm(g, x, w, b, eps, tag):
    mean = g.node("ReduceMean", [x], {"axes": [-1]})
    diff = g.node("Sub", [x, mean])
    pw = g.node("Pow", [diff, g.const(f"{tag}.two", np.array([2.0], np.float32))])
    var = g.node("ReduceMean", [pw], {"axes": [-1]})
    ve = g.node("Add", [var, g.const(f"{tag}.eps", np.array([eps], np.float32))])
    sd = g.node("Sqrt", [ve])
    nm = g.node("Div", [diff, sd])
    mu = g.node("Mul", [nm, g.const(f"{tag}.w", w)])
    return g.node("Identity", [g.node("Add", [mu, g.const(f"{tag}.b", b)])])


def svtr_graph(w, head_w=None, head_b=None, variant=None):
    """Nodes and tensors of a recognition graph from the flattened features [B, D, T] and the
    shortcut [B, D, 1, T] (graph inputs) to the head's Softmax, built as PP-OCRv6_small_rec
    lays its tail out: Transpose.0, blocks of LayerNorm sub-graph, MatMul + Add, Reshape
    [0,-1,3,H,hd], Transpose [2,0,3,1,4], Slice + Squeeze per q/k/v, Mul(scale) and a Reshape to q's own shape, Transpose
    [0,1,3,2], MatMul, Softmax(axis 3), MatMul, Transpose [0,2,1,3], Reshape [0,-1,D],
    MatMul + Add, residual Add, LayerNorm, MatMul + Add, Sigmoid, Mul, MatMul + Add, residual
    Add; then the final LayerNorm, Reshape [0,1,-1,D] (after its shape arithmetic),
    Transpose [0,3,1,2], Add(shortcut), Squeeze(axis 2), Transpose [0,2,1] and the head.

    `variant` alters the first block's attention or the node order, for the graph search's
    refusals: "gather" (q, k, v by Gather instead of Slice + Squeeze; still the pattern),
    "mask_add" (an Add on the scores), "softmax_queries" (Softmax over axis 2),
    "k_perm" (k transposed [0,2,1,3]), "k_as_v" (MatMul(p, k)), "scale_twice" (q scaled
    twice), "head_first" (the head's nodes listed first and the list ending inside the
    first attention), "one_input_matmul" (a one-input MatMul after the last Transpose)."""
    g = _G()
    x = g.node("Transpose", ["feat"], {"perm": [0, 2, 1]})
    i64 = lambda *v: np.array(v, np.int64)
    for bi, b in enumerate(w["blocks"]):
        t = f"b{bi}"
        y = _layer_norm(g, x, b["ln1_w"], b["ln1_b"], b["ln1_eps"], f"{t}.ln1")
        qkv = g.node("Add", [g.node("MatMul", [y, g.const(f"{t}.qkv.w", b["qkv_w"])]), g.const(f"{t}.qkv.b", b["qkv_b"])])
        r5 = g.node("Reshape", [qkv, g.const(f"{t}.shape5", i64(0, -1, 3, HEADS, DIM // HEADS))])
        tr = g.node("Transpose", [r5], {"perm": [2, 0, 3, 1, 4]})
        var = variant if bi == 0 else None
        parts = []
        for j in range(3):
            if var == "gather":
                parts.append(g.node("Gather", [tr, g.const(f"{t}.g{j}", np.array(j, np.int64))], {"axis": 0}))
                continue
            sl = g.node("Slice", [tr, g.const(f"{t}.s{j}", i64(j)), g.const(f"{t}.e{j}", i64(j + 1)),
                                  g.const(f"{t}.a{j}", i64(0)), g.const(f"{t}.p{j}", i64(1))])
            parts.append(g.node("Squeeze", [sl], {"axes": [0]}))
        q = g.node("Mul", [parts[0], g.const(f"{t}.scale", np.array([SCALE], np.float32))])
        if var == "scale_twice":
            q = g.node("Mul", [q, g.const(f"{t}.scale2", np.array([2.0], np.float32))])
        q = g.node("Reshape", [q, g.node("Shape", [parts[0]])])
        kt = g.node("Transpose", [parts[1]], {"perm": [0, 2, 1, 3] if var == "k_perm" else [0, 1, 3, 2]})
        sc = g.node("MatMul", [q, kt])
        if var == "mask_add":
            sc = g.node("Add", [sc, g.const(f"{t}.mask", np.zeros((1,), np.float32))])
        p = g.node("Softmax", [sc], {"axis": 2 if var == "softmax_queries" else 3})
        o = g.node("MatMul", [p, parts[1] if var == "k_as_v" else parts[2]])
        o = g.node("Reshape", [g.node("Transpose", [o], {"perm": [0, 2, 1, 3]}), g.const(f"{t}.shape3", i64(0, -1, DIM))])
        if bi == 0:
            att_end = len(g.nodes)  # nodes of the graph up to the first attention's output
        pr = g.node("Add", [g.node("MatMul", [o, g.const(f"{t}.proj.w", b["proj_w"])]), g.const(f"{t}.proj.b", b["proj_b"])])
        x = g.node("Add", [x, pr])
        y = _layer_norm(g, x, b["ln2_w"], b["ln2_b"], b["ln2_eps"], f"{t}.ln2")
        h = g.node("Add", [g.node("MatMul", [y, g.const(f"{t}.fc1.w", b["fc1_w"])]), g.const(f"{t}.fc1.b", b["fc1_b"])])
        hs = g.node("Mul", [h, g.node("Sigmoid", [h])])
        f2 = g.node("Add", [g.node("MatMul", [hs, g.const(f"{t}.fc2.w", b["fc2_w"])]), g.const(f"{t}.fc2.b", b["fc2_b"])])
        x = g.node("Add", [x, f2])
    z = _layer_norm(g, x, w["lnf_w"], w["lnf_b"], w["lnf_eps"], "lnf")
    shp = g.node("Concat", [g.const("c0", i64(0)), g.const("c1", i64(1)), g.const("cm1", i64(-1)),
                            g.const("cd", i64(DIM))], {"axis": 0})
    z = g.node("Transpose", [g.node("Reshape", [z, shp])], {"perm": [0, 3, 1, 2]})
    z = g.node("Squeeze", [g.node("Add", [z, "shortcut"])], {"axes": [2]})
    z = g.node("Transpose", [z], {"perm": [0, 2, 1]})
    last_transpose = len(g.nodes) - 1
    if variant == "one_input_matmul":
        g.node("MatMul", [z])
    outputs = [z]
    if head_w is not None:
        lg = g.node("Add", [g.node("MatMul", [z, g.const("head.w", head_w)]), g.const("head.b", head_b)])
        outputs = [g.node("Softmax", [lg], {"axis": 2})]
    nodes = g.nodes
    if variant == "head_first":
        # the head (its MatMul, Add, Softmax) and the Transpose feeding it first, then the
        # graph's first nodes up to the first attention's output: no weighted MatMul follows it
        nodes = nodes[-3:] + [nodes[last_transpose]] + nodes[:att_end]
    return {"inputs": ["feat", "shortcut"], "outputs": outputs, "nodes": nodes}, g.tensors


def write_model(path, graph, tensors):
    """A safetensors file holding `tensors` and the graph in its metadata."""
    hdr, blobs, off = {}, [], 0
    for name, a in tensors.items():
        dt = {np.dtype(np.float32): "F32", np.dtype(np.int64): "I64"}[a.dtype]
        b = a.tobytes()
        hdr[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    hdr["__metadata__"] = {"graph": json.dumps(graph)}
    h = json.dumps(hdr).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


# ---------------------------------------------------------------- graph interpreter
def _softmax(x, axis):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(axis=axis, keepdims=True))
    return (e / e.sum(axis=axis, keepdims=True)).astype(np.float32)


def run_graph(nodes, tensors, env, until=None):
    """Evaluates, in graph order, every node whose inputs are known (env: activations by
    name, tensors: weights by name), with ONNX semantics in float32 (MatMul products summed
    in float64 and rounded once, softmax in float64); stops after the node producing
    `until`.  Returns env."""
    env = dict(env)

    def val(n):
        return env[n] if n in env else tensors[n]

    for nd in nodes:
        ins = nd["inputs"]
        if not all((i in env) or (i in tensors) for i in ins):
            continue
        op, a, at = nd["op"], [val(i) for i in ins], nd.get("attrs", {})
        if op == "Identity":
            r = a[0]
        elif op == "Transpose":
            r = np.transpose(a[0], at["perm"])
        elif op == "Reshape":
            shape = [int(s) for s in a[1]]
            shape = [a[0].shape[i] if s == 0 else s for i, s in enumerate(shape)]
            r = a[0].reshape(shape)
        elif op == "Shape":
            r = np.array(a[0].shape, np.int64)
        elif op == "Slice":
            starts, ends = a[1], a[2]
            axes = a[3] if len(a) > 3 else np.arange(len(starts))
            steps = a[4] if len(a) > 4 else np.ones(len(starts), np.int64)
            sl = [slice(None)] * a[0].ndim
            for s, e, ax, st in zip(starts, ends, axes, steps):
                sl[int(ax)] = slice(int(s), int(min(e, a[0].shape[int(ax)])), int(st))
            r = a[0][tuple(sl)]
        elif op == "Squeeze":
            r = np.squeeze(a[0], axis=tuple(at["axes"]))
        elif op == "Unsqueeze":
            r = np.expand_dims(a[0], tuple(at["axes"]))
        elif op == "Concat":
            r = np.concatenate(a, axis=at["axis"])
        elif op in ("Add", "Sub", "Mul", "Div", "Pow"):
            f = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide, "Pow": np.power}[op]
            r = f(a[0], a[1])
            r = r.astype(a[0].dtype if a[0].dtype == a[1].dtype else np.float32)
        elif op == "Sqrt":
            r = np.sqrt(a[0])
        elif op == "ReduceMean":
            r = a[0].astype(np.float64).mean(axis=tuple(at["axes"]), keepdims=bool(at.get("keepdims", 1)))
            r = r.astype(np.float32)
        elif op == "MatMul":
            r = np.matmul(a[0].astype(np.float64), a[1].astype(np.float64)).astype(np.float32)
        elif op == "Softmax":
            r = _softmax(a[0], at.get("axis", -1))
        elif op == "Sigmoid":
            r = (1.0 / (1.0 + np.exp(-a[0].astype(np.float64)))).astype(np.float32)
        else:
            raise NotImplementedError(op)
        env[nd["outputs"][0]] = r
        if until is not None and nd["outputs"][0] == until:
            break
    return env
