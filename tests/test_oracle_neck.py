"""The oracle of the SVTR neck tail (oracle.py svtr_neck and its pieces), pinned on the CPU:
LayerNorm and sigmoid against float64 closed forms, the attention on cases with known
answers, the whole tail against a node-by-node interpretation of a graph with the real
model's layout (and, when the reference's model files are present, the real graph with its
real weights), plus the structural properties the GPU tests rely on.  Also the graph search
of the model-file constructor, through the host-only parser driver."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from neck_common import (DIM, HEADS, SCALE, lines_of, neck_weights, oracle_neck, run_graph, svtr_graph,
                         write_model)

REF_MODEL = "/root/reference/models/PP-OCRv6_small_rec.safetensors"


def test_layer_norm_matches_the_closed_form(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, DIM)) * 3 + 1).astype(np.float32)
    w = rng.standard_normal(DIM).astype(np.float32)
    b = rng.standard_normal(DIM).astype(np.float32)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(1, keepdims=True) + 1e-5) * w + b
    for avx in (True, False):
        got = orc.layer_norm_rows(x, w, b, 1e-5, use_avx2=avx)
        assert np.abs(got - ref).max() < 2e-6 * np.abs(ref).max()
    # a row of equal values normalises to b exactly
    got = orc.layer_norm_rows(np.full((1, DIM), 7.0, np.float32), w, b, 1e-5)
    assert np.array_equal(got[0], b)


def test_sigmoid_matches_the_closed_form(orc):
    x = np.linspace(-30, 30, 4001).astype(np.float32)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    got = orc.sigmoid(x)
    assert np.abs(got - ref).max() <= 4e-7 * 1.0 and np.all(np.abs(got - ref) <= 1e-6 * ref + 1e-30)
    assert orc.sigmoid(np.zeros(8, np.float32))[0] == 0.5


def test_attention_known_answers(orc):
    rng = np.random.default_rng(2)
    # one token: the softmax is [1], the output is v
    qkv = rng.standard_normal((1, 3 * DIM)).astype(np.float32)
    assert np.array_equal(orc.attention_line(qkv, HEADS, SCALE), qkv[:, 2 * DIM:])
    # equal keys: uniform weights, the output is the mean of v
    qkv = rng.standard_normal((9, 3 * DIM)).astype(np.float32)
    qkv[:, DIM:2 * DIM] = qkv[0, DIM:2 * DIM]
    got = orc.attention_line(qkv, HEADS, SCALE)
    assert np.abs(got - qkv[:, 2 * DIM:].astype(np.float64).mean(0)).max() < 1e-6
    # against float64 scaled dot-product attention per head
    qkv = (rng.standard_normal((37, 3 * DIM)) * 2).astype(np.float32)
    got = orc.attention_line(qkv, HEADS, SCALE)
    x = qkv.astype(np.float64).reshape(37, 3, HEADS, DIM // HEADS)
    ref = np.empty((37, HEADS, DIM // HEADS))
    for h in range(HEADS):
        s = (x[:, 0, h] * float(SCALE)) @ x[:, 1, h].T
        p = np.exp(s - s.max(1, keepdims=True))
        ref[:, h] = (p / p.sum(1, keepdims=True)) @ x[:, 2, h]
    assert np.abs(got - ref.reshape(37, DIM)).max() < 2e-6


def _inputs(lengths, seed=3):
    rng = np.random.default_rng(seed)
    off = lines_of(lengths)
    m = int(off[-1])
    return rng.standard_normal((m, DIM)).astype(np.float32), rng.standard_normal((m, DIM)).astype(np.float32), off


def test_neck_lines_are_independent_and_tokens_equivariant(orc):
    w = neck_weights()
    x, sc, off = _inputs([5, 17, 1, 30])
    whole = oracle_neck(orc, w, x, sc, off)
    for b in range(4):
        t0, t1 = off[b], off[b + 1]
        alone = oracle_neck(orc, w, x[t0:t1], sc[t0:t1], np.array([0, t1 - t0]))
        assert np.array_equal(alone, whole[t0:t1])
    # permuting the tokens of a line permutes its outputs (no positional term in the tail)
    perm = np.random.default_rng(4).permutation(30)
    t0 = off[3]
    xp, sp = x.copy(), sc.copy()
    xp[t0:] = x[t0:][perm]
    sp[t0:] = sc[t0:][perm]
    got = oracle_neck(orc, w, xp, sp, off)
    assert np.abs(got[t0:] - whole[t0:][perm]).max() < 1e-5


def _interpret(nodes, tensors, x, sc, off, feat="feat", short="shortcut", out=None):
    rows = []
    for b in range(off.size - 1):
        t0, t1 = off[b], off[b + 1]
        env = run_graph(nodes, tensors, {feat: x[t0:t1].T[None].copy(), short: sc[t0:t1].T[None, :, None, :].copy()},
                        until=out)
        rows.append(env[out][0])
    return np.concatenate(rows)


def test_oracle_neck_equals_the_graph_interpreted_node_by_node(orc):
    """The oracle's tail against an ONNX-semantics interpretation of a graph laid out as
    PP-OCRv6_small_rec's (qkv column order from Reshape [0,-1,3,H,hd] + Transpose
    [2,0,3,1,4], heads concatenated by Transpose [0,2,1,3], residuals, swish, the final
    LayerNorm and the shortcut)."""
    w = neck_weights()
    x, sc, off = _inputs([1, 12, 40])
    graph, tensors = svtr_graph(w)
    got = oracle_neck(orc, w, x, sc, off)
    ref = _interpret(graph["nodes"], tensors, x, sc, off, out=graph["outputs"][0])
    assert np.abs(got - ref).max() < 2e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.skipif(not os.path.exists(REF_MODEL), reason="the reference's model files are not here")
def test_oracle_neck_on_the_real_model_graph(orc):
    """The real PP-OCRv6_small_rec: its graph from the flatten output and the shortcut to
    Transpose.8, interpreted node by node with its own weights, equals the oracle's tail
    with the weights the graph search names; and the synthetic graph of the GPU tests has
    the real tail's node sequence."""
    import json
    from safetensors.numpy import load_file
    tensors = load_file(REF_MODEL)
    meta = json.loads(open(REF_MODEL, "rb").read(8 + int.from_bytes(open(REF_MODEL, "rb").read(8), "little"))[8:])
    graph = json.loads(meta["__metadata__"]["graph"])
    names = _parse_neck(REF_MODEL)
    blocks = []
    for b in names["blocks"]:
        d = {k: tensors[v] for k, v in b.items() if not k.endswith("eps")}
        d["ln1_eps"], d["ln2_eps"] = b["ln1_eps"], b["ln2_eps"]
        blocks.append(d)
    x, sc, off = _inputs([9, 40])
    got = orc.svtr_neck(x, sc, off, blocks, tensors[names["lnf_w"]], tensors[names["lnf_b"]], names["lnf_eps"],
                        HEADS, names["scale"])
    t8 = next(n for n in graph["nodes"] if n["name"] == "Transpose.8")["outputs"][0]
    feat, short = names["input"], names["shortcut"]
    # the flatten output [1, D, T] and the shortcut [1, D, 1, T] are where the tail starts
    ref = []
    for b in range(off.size - 1):
        t0, t1 = off[b], off[b + 1]
        env = {feat: x[t0:t1].T[None].copy(), short: sc[t0:t1].T[None, :, None, :].copy()}
        # shapes the graph computes from the feature map before the flatten
        env["p2o.pd_op.add.65.0"] = x[t0:t1].T[None, :, None, :].copy()
        env = run_graph(graph["nodes"], tensors, env, until=t8)
        ref.append(env[t8][0])
    ref = np.concatenate(ref)
    assert np.abs(got - ref).max() < 2e-5 * max(1.0, np.abs(ref).max())
    # node sequence of the synthetic graph = the real tail's (Identity and shape arithmetic aside)
    skip = {"Identity", "Shape", "Unsqueeze", "Concat", "Slice", "Squeeze"}
    nodes = graph["nodes"]
    i0 = next(i for i, n in enumerate(nodes) if n["op"] == "Transpose" and n["inputs"][0] == feat)
    i1 = next(i for i, n in enumerate(nodes) if n["name"] == "Transpose.8")
    real = [n["op"] for n in nodes[i0:i1 + 1] if n["op"] not in skip]
    syn_graph, _ = svtr_graph(neck_weights())
    syn = [n["op"] for n in syn_graph["nodes"] if n["op"] not in skip]
    assert syn == real


def _parse_neck(path):
    """The neck the library's graph search finds in a model file (host-only driver)."""
    exe = os.path.join(ROOT, "rust-ppocrv6_amd", "lib", "_asan", "parser_check")
    if not os.path.exists(exe):
        subprocess.run(["make", "-C", os.path.join(ROOT, "rust-ppocrv6_amd", "csrc"), "asan"], check=True,
                       capture_output=True)
    out = subprocess.run([exe, "--neck", path], check=True, capture_output=True, text=True).stdout.splitlines()
    head = out[0].split()
    assert head[0] == "neck", out
    kv = lambda key, k=1: head[head.index(key) + k]
    res = {"dim": int(kv("dim")), "heads": int(kv("heads")), "hidden": int(kv("hidden")),
           "scale": np.float32(kv("scale")), "lnf_w": kv("lnf"), "lnf_b": kv("lnf", 2), "lnf_eps": float(kv("eps")),
           "input": kv("input"), "shortcut": kv("shortcut"), "blocks": []}
    for line in out[1:]:
        if not line.startswith("  block"):
            continue
        t = line.split()
        g = lambda key, k=1: t[t.index(key) + k]
        res["blocks"].append({"ln1_w": g("ln1"), "ln1_b": g("ln1", 2), "ln1_eps": float(g("ln1", 3)),
                              "qkv_w": g("qkv"), "qkv_b": g("qkv", 2), "proj_w": g("proj"), "proj_b": g("proj", 2),
                              "ln2_w": g("ln2"), "ln2_b": g("ln2", 2), "ln2_eps": float(g("ln2", 3)),
                              "fc1_w": g("fc1"), "fc1_b": g("fc1", 2), "fc2_w": g("fc2"), "fc2_b": g("fc2", 2)})
    return res


def test_graph_search_finds_the_synthetic_tail(tmp_path):
    w = neck_weights()
    head_w = np.random.default_rng(5).standard_normal((DIM, 64)).astype(np.float32) * 0.05
    graph, tensors = svtr_graph(w, head_w, np.zeros(64, np.float32))
    path = str(tmp_path / "svtr.safetensors")
    write_model(path, graph, tensors)
    got = _parse_neck(path)
    assert (got["dim"], got["heads"], got["hidden"], len(got["blocks"])) == (DIM, HEADS, 240, 2)
    assert got["scale"] == SCALE and got["lnf_w"] == "lnf.w" and got["lnf_eps"] == pytest.approx(1e-6)
    assert got["blocks"][1]["fc2_w"] == "b1.fc2.w" and got["blocks"][0]["qkv_b"] == "b0.qkv.b"
    assert got["input"] == "feat" and got["shortcut"] == "shortcut"


@pytest.mark.parametrize("variant,msg", [
    ("gather", None),
    ("mask_add", "node outside the attention pattern"),
    ("softmax_queries", "Softmax other than over the keys"),
    ("k_perm", "unexpected Transpose"),
    ("k_as_v", "MatMul other than (q * scale) k^T or p v"),
    ("scale_twice", "Mul other than q by a scalar constant"),
    ("head_first", "no projection MatMul after it"),
    ("one_input_matmul", "the tail does not feed the head's MatMul"),
])
def test_graph_search_refuses_other_attention_structures(tmp_path, variant, msg):
    """The graph search takes exactly the attention the kernels compute, softmax(q * scale *
    k^T) v per head, with each node's inputs traced to the q, k and v parts of the qkv
    Reshape: an Add on the scores, a Softmax over the queries, k transposed otherwise, k
    used as v or a second scaling refuse the file (PPOCR_ERR_MODEL with the node named).
    q, k and v taken by Gather is the same computation and is accepted.  The structures of
    a head listed before the tail (the attention scan then runs to the end of the node list)
    and a one-input MatMul after the last Transpose are refused without reading past a
    list; the driver is the AddressSanitizer / UBSan build, so any such read fails it."""
    w = neck_weights()
    head_w = np.random.default_rng(5).standard_normal((DIM, 64)).astype(np.float32) * 0.05
    graph, tensors = svtr_graph(w, head_w, np.zeros(64, np.float32), variant=variant)
    path = str(tmp_path / f"svtr_{variant}.safetensors")
    write_model(path, graph, tensors)
    if msg is None:
        got = _parse_neck(path)
        assert (got["heads"], len(got["blocks"])) == (HEADS, 2) and got["scale"] == SCALE
        return
    exe = os.path.join(ROOT, "rust-ppocrv6_amd", "lib", "_asan", "parser_check")
    out = subprocess.run([exe, "--neck", path], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr[-3000:]
    assert "runtime error" not in out.stderr and "Sanitizer" not in out.stderr, out.stderr[-3000:]
    assert "necks 0" in out.stdout and msg in out.stdout, out.stdout


@pytest.mark.skipif(not os.path.exists(REF_MODEL), reason="the reference's model files are not here")
def test_graph_search_on_the_real_models():
    got = _parse_neck(REF_MODEL)
    assert (got["dim"], got["heads"], got["hidden"], len(got["blocks"])) == (120, 8, 240, 2)
    assert got["blocks"][0]["qkv_w"] == "linear_0.w_0" and got["blocks"][1]["fc2_w"] == "linear_7.w_0"
    assert got["lnf_eps"] == pytest.approx(1e-6) and got["blocks"][0]["ln1_eps"] == pytest.approx(1e-5)
    assert abs(got["scale"] - 15 ** -0.5) < 1e-7
    tiny = REF_MODEL.replace("small", "tiny")
    exe = os.path.join(ROOT, "rust-ppocrv6_amd", "lib", "_asan", "parser_check")
    out = subprocess.run([exe, "--neck", tiny], check=True, capture_output=True, text=True).stdout
    assert "no LayerNorm sub-graph" in out and "necks 0" in out
