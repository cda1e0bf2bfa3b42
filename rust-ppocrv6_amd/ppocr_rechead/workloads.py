"""Seeded synthetic inputs of the recognition head's five benchmark workloads.

The reference has no input generator (its tests use sin/cos patterns), so the inputs
are defined here: numpy's PCG64 generator, one stream per tensor, float32 normals.

    single_line   1 line  x T=120 (rec_small on a 1x3x48x960 crop), INT8 head
    a4_page       29 lines, widths uniform on {160, 168, ..., 960}, T_i = W_i / 8
    dense_256     256 lines x T=120 (m = 30720), INT8 head
    fp32_64       64 lines x T=120 (m = 7680), FP32 head
    stress_1024   1024 lines x T=240 (m = 245760), INT8 head with zero rows, +-5
                  outliers, 1% activation rows x50 and 2% rows built to near-tie

Weights W^T [18710, 120] ~ N(0, 0.05^2), bias ~ N(0, 0.01^2), activations ~ N(0, 1).
"""
import numpy as np

N_CLASSES = 18710
K_DIM = 120
SEED_W = 0x5EED0001
SEED_BIAS = 0x5EED0002
SEED_A = 0x5EED0100

WORKLOADS = ("single_line", "a4_page", "dense_256", "fp32_64", "stress_1024")


def weights(n=N_CLASSES, k=K_DIM, stress=False):
    """W^T f32 [n, k] and bias f32 [n]."""
    rng = np.random.default_rng(SEED_W)
    w_t = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    bias = (np.random.default_rng(SEED_BIAS).standard_normal(n, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    if stress:
        srng = np.random.default_rng(SEED_W + 0x100)
        rows = srng.permutation(n)
        nz = max(1, n // 200)
        zero_rows = np.sort(rows[:nz])
        out_rows = np.sort(rows[nz:2 * nz])
        w_t[zero_rows] = 0.0
        cols = srng.integers(0, k, out_rows.size)
        signs = np.where(srng.integers(0, 2, out_rows.size) == 0, -5.0, 5.0).astype(np.float32)
        w_t[out_rows, cols] = signs
    return w_t, bias


def line_offsets(lengths):
    off = np.zeros(len(lengths) + 1, np.int64)
    off[1:] = np.cumsum(np.asarray(lengths, dtype=np.int64))
    return off


def lines_for(name):
    if name == "single_line":
        return [120]
    if name == "a4_page":
        rng = np.random.default_rng(SEED_A + 1)
        widths = 160 + 8 * rng.integers(0, 101, 29)
        return [int(w // 8) for w in widths]
    if name == "dense_256":
        return [120] * 256
    if name == "fp32_64":
        return [120] * 64
    if name == "stress_1024":
        return [240] * 1024
    raise ValueError(f"unknown workload {name!r}")


def activations(name, lengths=None, k=K_DIM):
    lengths = lines_for(name) if lengths is None else lengths
    m = int(sum(lengths))
    rng = np.random.default_rng(SEED_A + WORKLOADS.index(name))
    a = rng.standard_normal((m, k), dtype=np.float32)
    return a


def make(name, pack=None, near_tie_fraction=0.02, scaled_fraction=0.01):
    """Build a workload.  `pack(w_t) -> (q, scales)` is the INT8 packer (needed by the
    stress workload to place near-ties on the dequantised weights)."""
    lengths = lines_for(name)
    w_t, bias = weights(stress=(name == "stress_1024"))
    a = activations(name, lengths)
    out = {"name": name, "a": a, "line_off": line_offsets(lengths), "w_t": w_t, "bias": bias,
           "quantized": name != "fp32_64"}
    if name == "stress_1024":
        if pack is None:
            raise ValueError("the stress workload needs a packer")
        q, scales = pack(w_t)
        out["q"], out["scales"] = q, scales
        m = a.shape[0]
        rng = np.random.default_rng(SEED_A + 0x40)
        perm = rng.permutation(m)
        n_scaled = int(round(scaled_fraction * m))
        n_tie = int(round(near_tie_fraction * m))
        scaled_rows = np.sort(perm[:n_scaled])
        tie_rows = np.sort(perm[n_scaled:n_scaled + n_tie])
        a[scaled_rows] *= np.float32(50.0)
        out["scaled_rows"] = scaled_rows
        out["tie_rows"] = make_near_ties(a, tie_rows, q, scales, bias, rng)
    return out


def make_near_ties(a, rows, q, scales, bias, rng, target_gap=(1e-7, 1e-5), chunk=1024):
    """Move each listed activation row along w~_c1 - w~_c2 (dequantised top-2 classes, in
    f64) until the top-2 logit gap is below 1e-5.  Returns the rows that achieved it."""
    wd_t = np.ascontiguousarray((q.astype(np.float64) * scales.astype(np.float64)[:, None]).T)
    b64 = bias.astype(np.float64)
    ok = []
    for s in range(0, rows.size, chunk):
        rr = rows[s:s + chunk]
        x = a[rr].astype(np.float64)
        lg = x @ wd_t + b64
        top2 = np.argpartition(-lg, 1, axis=1)[:, :2]
        r_ix = np.arange(rr.size)
        first = lg[r_ix, top2[:, 0]] >= lg[r_ix, top2[:, 1]]
        c1 = np.where(first, top2[:, 0], top2[:, 1])
        c2 = np.where(first, top2[:, 1], top2[:, 0])
        d = wd_t[:, c1].T - wd_t[:, c2].T
        dd = (d * d).sum(axis=1)
        g = lg[r_ix, c1] - lg[r_ix, c2]
        tgt = rng.uniform(*target_gap, rr.size)
        step = np.where(dd > 0, (g - tgt) / np.where(dd > 0, dd, 1.0), 0.0)
        xn = (x - step[:, None] * d).astype(np.float32)
        l2 = xn.astype(np.float64) @ wd_t + b64
        o = np.argpartition(-l2, 1, axis=1)[:, :2]
        keep = (dd > 0) & (np.abs(l2[r_ix, c1] - l2[r_ix, c2]) <= 1e-5)
        keep &= ((o[:, 0] == c1) & (o[:, 1] == c2)) | ((o[:, 0] == c2) & (o[:, 1] == c1))
        a[rr[keep]] = xn[keep]
        ok.extend(rr[keep].tolist())
    return np.asarray(sorted(ok), dtype=np.int64)


NECK_DIM, NECK_HEADS, NECK_HIDDEN = 120, 8, 240
SEED_NECK = 0x5EED0300


def neck_weights(seed=SEED_NECK, blocks=2):
    """Weights of the SVTR tail before the head (ppocr_rn_block_t fields per block, plus the
    final LayerNorm), seeded normals with the statistics of PP-OCRv6_small_rec's tail:
    LayerNorm weights ~1 +- 0.2 (final ~3 +- 1.7), MatMul weights 0.045-0.1, biases
    0.03-0.17."""
    rng = np.random.default_rng(seed)
    d, hd = NECK_DIM, NECK_HIDDEN

    def f(*shape, s=1.0, mu=0.0):
        return (mu + s * rng.standard_normal(shape)).astype(np.float32)

    bl = []
    for _ in range(blocks):
        bl.append({"ln1_w": f(d, s=0.2, mu=1.0), "ln1_b": f(d, s=0.3), "ln1_eps": 1e-5,
                   "qkv_w": f(d, 3 * d, s=0.08), "qkv_b": f(3 * d, s=0.16),
                   "proj_w": f(d, d, s=0.05), "proj_b": f(d, s=0.03),
                   "ln2_w": f(d, s=0.2, mu=1.0), "ln2_b": f(d, s=0.3), "ln2_eps": 1e-5,
                   "fc1_w": f(d, hd, s=0.1), "fc1_b": f(hd, s=0.07),
                   "fc2_w": f(hd, d, s=0.045), "fc2_b": f(d, s=0.08)})
    return {"blocks": bl, "lnf_w": f(d, s=1.7, mu=3.0), "lnf_b": f(d, s=0.6, mu=-0.5), "lnf_eps": 1e-6}


def neck_kernel_work(steps_of, blocks=2):
    """Algorithmic work of each kernel of the tail's forward on token rows (row layout), in
    launch order: (name, flops, HBM bytes).  Flops: 2 per multiply-add of each MatMul and of
    the attention's scores and weighted values (sum over lines of 4 T^2 D); bytes: fp32 rows
    read and written once (the weights, under 0.3 MB per block, are left out)."""
    d, h = NECK_DIM, NECK_HIDDEN
    steps_of = np.asarray(steps_of, np.int64)
    m = int(steps_of.sum())
    row = 4 * d * m  # bytes of one [m][d] fp32 tensor
    out = []
    for b in range(blocks):
        last = b + 1 == blocks
        out += [("ln1_qkv", 2.0 * m * d * 3 * d, row + 3 * row),
                ("attention", 4.0 * d * float((steps_of.astype(np.float64) ** 2).sum()), 3 * row + row),
                ("proj_residual", 2.0 * m * d * d, 3 * row),
                ("mlp_final_ln_shortcut" if last else "mlp", 2.0 * m * (d * h + h * d), (3 if last else 2) * row)]
    return out


def neck_flops_per_row(steps, blocks=2):
    """Algorithmic FLOPs of the tail per token row of a line of `steps` tokens: the four
    MatMuls of each block (2 D 3D + 2 D D + 2 D H + 2 H D) and its attention (2 steps D for
    the scores, 2 steps D for the weighted values)."""
    d, h = NECK_DIM, NECK_HIDDEN
    return blocks * (2 * d * 3 * d + 2 * d * d + 2 * d * h + 2 * h * d + 4 * steps * d)

