"""GPU parity of the SVTR neck tail (ppocr_rn_*) against the oracle's restatement
(oracle.py svtr_neck: the reference's LayerNorm and sigmoid, softmax over the keys,
correctly rounded MatMuls), on ragged batches of lines; the layouts, the model-file
constructor and the device entry point against each other bit for bit; and the neck
feeding the head against the oracle's neck feeding the oracle's head.

The bar: the kernels sum the MatMuls and the attention in another order than the oracle
(MFMA on fp16 halves of both operands or on fp32, an online softmax), so the tail's outputs
(magnitude up to ~30 with the final LayerNorm's weights) may differ by a few fp32 roundings
of the sums they pass through; they are held to 1e-4 absolute + 1e-5 relative."""
import numpy as np
import pytest

from neck_common import DIM, lines_of, neck_weights, oracle_neck, rows_to_cf, svtr_graph, write_model

pytestmark = pytest.mark.gpu


def _make(rh, w):
    return rh.RecNeck(w["blocks"], w["lnf_w"], w["lnf_b"], w["lnf_eps"])


def _inputs(lengths, seed=11, scale=1.5):
    rng = np.random.default_rng(seed)
    off = lines_of(lengths)
    m = int(off[-1])
    return ((rng.standard_normal((m, DIM)) * scale).astype(np.float32), rng.standard_normal((m, DIM)).astype(np.float32),
            off)


def _check(got, ref, label):
    err = np.abs(got - ref)
    bar = 1e-4 + 1e-5 * np.abs(ref)
    print(f"{label}: max|diff| {err.max():.3e}, worst diff/bar {np.max(err / bar):.3f}, max|ref| {np.abs(ref).max():.2f}",
          flush=True)
    assert np.all(err <= bar), label


@pytest.mark.parametrize("lengths", [[1], [7, 40, 1, 120, 3], [240, 240, 97], [16, 17, 255, 256, 31],
                                     [300, 257, 5]])
def test_neck_matches_the_oracle(orc, rh, lengths):
    w = neck_weights()
    neck = _make(rh, w)
    x, sc, off = _inputs(lengths)
    got = neck.forward(x, sc, off)
    _check(got, oracle_neck(orc, w, x, sc, off), f"neck lines {lengths}")
    # the channels-first layout (the graph's [1, D, T] per line) gives the same bits
    got_cf = neck.forward(rows_to_cf(x, off), rows_to_cf(sc, off), off, layout=rh.NECK_CHANNELS_FIRST)
    assert np.array_equal(got_cf, got)
    neck.close()


def test_neck_large_batch_against_the_oracle_on_sampled_lines(orc, rh):
    """64 lines of the longest crops (T = 240): the whole batch on the GPU, the oracle on
    six of its lines (lines are independent, so a line's outputs do not depend on the
    others)."""
    w = neck_weights(seed=9)
    neck = _make(rh, w)
    lengths = [240] * 60 + [1, 2, 120, 239]
    x, sc, off = _inputs(lengths, seed=12)
    got = neck.forward(x, sc, off)
    for b in (0, 31, 59, 60, 62, 63):
        t0, t1 = off[b], off[b + 1]
        ref = oracle_neck(orc, w, x[t0:t1], sc[t0:t1], np.array([0, t1 - t0]))
        _check(got[t0:t1], ref, f"large batch line {b}")
    neck.close()


def test_neck_matmul_arithmetic_follows_the_weight_bounds(orc, rh):
    """The model's weights bound every MatMul operand far inside fp16's range (LayerNorm
    outputs, attention outputs no larger than the value rows, swish no larger than its
    input), so the MatMuls run on fp16 halves; an fc1 weight 2000 times larger bounds fc2's
    input beyond the limit (16384) and the tail keeps fp32 products.  Both against the
    oracle at the same bar."""
    w = neck_weights(seed=41)
    neck = _make(rh, w)
    assert neck.gemm_halves
    x, sc, off = _inputs([37, 120, 5], seed=16)
    _check(neck.forward(x, sc, off), oracle_neck(orc, w, x, sc, off), "fp16 halves")
    neck.close()
    big = {**w, "blocks": [dict(b) for b in w["blocks"]]}
    big["blocks"][1]["fc1_w"] = (big["blocks"][1]["fc1_w"] * np.float32(2000.0)).astype(np.float32)
    neck = _make(rh, big)
    assert not neck.gemm_halves
    _check(neck.forward(x, sc, off), oracle_neck(orc, big, x, sc, off), "fp32 products")
    neck.close()


def test_neck_token_permutation_and_line_independence(rh):
    """No positional term in the tail: permuting a line's tokens permutes its outputs, and
    a line's outputs do not depend on the other lines of the batch."""
    w = neck_weights(seed=3)
    neck = _make(rh, w)
    x, sc, off = _inputs([50, 77, 13], seed=13)
    whole = neck.forward(x, sc, off)
    perm = np.random.default_rng(5).permutation(77)
    t0, t1 = off[1], off[2]
    xp, sp = x.copy(), sc.copy()
    xp[t0:t1], sp[t0:t1] = x[t0:t1][perm], sc[t0:t1][perm]
    got = neck.forward(xp, sp, off)
    assert np.abs(got[t0:t1] - whole[t0:t1][perm]).max() < 1e-4
    assert np.array_equal(got[:t0], whole[:t0]) and np.array_equal(got[t1:], whole[t1:])
    alone = neck.forward(x[t0:t1], sc[t0:t1], np.array([0, t1 - t0]))
    assert np.array_equal(alone, whole[t0:t1])
    neck.close()


def test_neck_from_a_model_file_and_the_device_entry(rh, tmp_path):
    """ppocr_rn_create_from_model on a file holding the tail in its graph builds the neck
    of ppocr_rn_create with the same weights (same bits out), and ppocr_rn_forward_dev with
    a caller workspace gives the host entry's bits."""
    from ppocr_rechead.hip import DeviceArray, synchronize
    w = neck_weights(seed=21)
    head_w = (np.random.default_rng(6).standard_normal((DIM, 96)) * 0.05).astype(np.float32)
    graph, tensors = svtr_graph(w, head_w, np.zeros(96, np.float32))
    path = str(tmp_path / "svtr.safetensors")
    write_model(path, graph, tensors)
    a = _make(rh, w)
    b = rh.RecNeck.from_model(path)
    assert (b.dim, b.heads, b.hidden, b.blocks) == (120, 8, 240, 2)
    x, sc, off = _inputs([33, 5, 64], seed=14)
    want = a.forward(x, sc, off)
    assert np.array_equal(b.forward(x, sc, off), want)
    L = rh._lib.lib()
    m = int(off[-1])
    dx, ds, doff = DeviceArray.from_numpy(x), DeviceArray.from_numpy(sc), DeviceArray.from_numpy(off)
    dout = DeviceArray((m, DIM), np.float32)
    wsb = a.workspace_bytes(m)
    dws = DeviceArray((wsb,), np.uint8)
    rh._check(L.ppocr_rn_forward_dev(a.handle, dx.p, ds.p, m, doff.p, 3, rh.NECK_ROWS, dout.p, dws.p, wsb, None))
    synchronize()
    assert np.array_equal(dout.numpy(), want)
    # too small a workspace is refused
    assert L.ppocr_rn_forward_dev(a.handle, dx.p, ds.p, m, doff.p, 3, rh.NECK_ROWS, dout.p, dws.p, wsb - 4,
                                  None) == rh.PPOCR_ERR_INVALID_ARG
    for d in (dx, ds, doff, dout, dws):
        d.free()
    a.close()
    b.close()


def test_neck_final_layernorm_with_unaligned_rows(rh):
    """The last block's fused kernel finishes the tail (final LayerNorm + shortcut) when the
    shortcut rows and the output are 16-byte aligned; otherwise a separate kernel does, with
    the same arithmetic: the same bits either way (rows 4 bytes off alignment)."""
    from ppocr_rechead.hip import DeviceArray, synchronize
    w = neck_weights(seed=23)
    neck = _make(rh, w)
    x, sc, off = _inputs([120, 61, 3], seed=17)
    m = int(off[-1])
    want = neck.forward(x, sc, off)
    L = rh._lib.lib()
    dx, doff = DeviceArray.from_numpy(x), DeviceArray.from_numpy(off)
    dsc = DeviceArray.from_numpy(np.concatenate([[0.0], sc.reshape(-1)]).astype(np.float32))
    dout = DeviceArray((m * DIM + 1,), np.float32)
    wsb = neck.workspace_bytes(m)
    dws = DeviceArray((wsb,), np.uint8)
    import ctypes
    off4 = lambda d: ctypes.c_void_p(d.p.value + 4)  # noqa: E731
    rh._check(L.ppocr_rn_forward_dev(neck.handle, dx.p, off4(dsc), m, doff.p, 3, rh.NECK_ROWS, off4(dout), dws.p, wsb,
                                     None))
    synchronize()
    got = dout.numpy()[1:].reshape(m, DIM)
    assert np.array_equal(got, want)
    for d in (dx, doff, dsc, dout, dws):
        d.free()
    neck.close()


def test_neck_then_head_against_the_oracle(orc, rh):
    """The tail feeding the head (PP-OCRv6_small_rec from the flatten output to the CTC
    sequences): argmax and sequences equal to the oracle's tail feeding the oracle's head
    except at top-2 logit gaps below 1e-4, max probabilities within 1e-4."""
    from gpu_common import check_argmax, top2_gap, f64_logits_q
    from ppocr_rechead import workloads as wl
    w = neck_weights(seed=31)
    neck = _make(rh, w)
    w_t, bias = wl.weights()
    q, s = orc.pack_int8(w_t)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    x, sc, off = _inputs([120, 64, 17], seed=15)
    feats = neck.forward(x, sc, off)
    got = head.decode(feats, off)
    ref_feats = oracle_neck(orc, w, x, sc, off)
    ref = orc.rechead_lines(ref_feats, off, q, s, bias)
    gap = top2_gap(f64_logits_q(ref_feats, q, s, bias))
    check_argmax(got["idx"], ref["idx"], gap, label="neck + head")
    assert np.abs(got["maxprob"] - ref["maxprob"]).max() < 1e-4
    neck.close()
    head.close()


def test_neck_argument_errors(rh, tmp_path):
    w = neck_weights()
    bad = [dict(b) for b in w["blocks"]]
    with pytest.raises(rh.OcrError) as e:
        rh.RecNeck(bad, w["lnf_w"], w["lnf_b"], w["lnf_eps"], heads=6)
    assert e.value.code == rh.PPOCR_ERR_INVALID_ARG and "unsupported geometry" in e.value.msg
    neck = _make(rh, w)
    x, sc, off = _inputs([4])
    with pytest.raises(rh.OcrError):
        neck.forward(x, sc, off, layout=7)
    neck.close()
    # a model without the tail (the head alone) is a model error
    graph, tensors = svtr_graph(w, np.zeros((DIM, 8), np.float32), np.zeros(8, np.float32))
    graph["nodes"] = [n for n in graph["nodes"] if n["op"] not in ("ReduceMean",)]
    path = str(tmp_path / "nohead.safetensors")
    write_model(path, graph, tensors)
    with pytest.raises(rh.OcrError) as e:
        rh.RecNeck.from_model(path)
    assert e.value.code == rh.PPOCR_ERR_MODEL
