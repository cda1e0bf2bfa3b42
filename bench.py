"""Recognition-head benchmark on one MI355X.

A step is one pass of the head over one batch already resident in HBM: the dense batch
of 256 text lines x T=120 (m = 30720 rows, k = 120, 18710 classes), INT8 weights, through
the fused projection + online softmax + argmax (never writing logits) and the CTC
collapse.  The metric is rows/s (rows = B*T).  The same JSON line carries the roofline of
the dominant kernel, the unfused variant (logits written to HBM, softmax, argmax, CTC)
and the CPU oracle (the C restatement of the reference's AVX2 INT8 path) timed on a
bounded sample on this host.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "rust-ppocrv6_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
MODE_NAMES = {0: "f32", 1: "bf16x1", 2: "bf16x2", 3: "bf16x3", 4: "f16x2", 5: "auto"}
TERMS = {1: 1, 2: 2, 3: 3, 4: 2}  # MFMA products per logit of an INT8 head in each mode


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default="dense_256")
    p.add_argument("--mode", type=int, default=2,
                   help="0 fp32 FMA, 1/2/3 bf16 terms (2: the headline), 4 two fp16 terms, 5 auto (the library's "
                        "default)")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-others", action="store_true", help="skip the other configurations")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", default="", help="fused|unfused|probs|neck (profiling runs)")
    p.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                   help="also run one device copy of this many MiB (counter calibration)")
    return p.parse_args()


def timed(fn, stream, steps, warmup):
    """Run fn() warmup times, then time `steps` calls with HIP events on `stream`."""
    from ppocr_rechead.hip import Event, synchronize
    for _ in range(warmup):
        fn()
    synchronize()
    e0, e1 = Event(), Event()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    e1.synchronize()
    wall = time.perf_counter() - t0
    synchronize()
    return e0.elapsed_ms(e1) / steps, wall / steps * 1e3


def ramp(fn, seconds=0.2):
    """Untimed passes of fn() for about `seconds` before a timed leg (beside its --warmup
    steps): the timed steps then start at the clocks this load holds, as the legs measured
    after them do (the first leg measured ~10% slow otherwise)."""
    from ppocr_rechead.hip import synchronize
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            fn()
        synchronize()


def traffic_from_profiles(kernel_key):
    """HBM bytes per launch measured with rocprofv3 --pmc (committed under profiles/)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel_key)
    except (OSError, ValueError):
        return None


def agreement(wk, q, s, ref, gpu):
    """The GPU step's results against the oracle's on the same batch, in the terms of the
    parity bar: argmax mismatches (each with its top-2 logit gap, from f64 logits of the
    dequantized weight), the largest maxprob difference, and per line whether the CTC
    sequences are identical, plus the largest score difference."""
    mis = np.nonzero(ref["idx"] != gpu["idx"])[0]
    gaps = []
    if mis.size:
        w = q.astype(np.float64) * s.astype(np.float64)[:, None]
        lg = wk["a"][mis].astype(np.float64) @ w.T + wk["bias"].astype(np.float64)
        top2 = np.sort(lg, axis=1)[:, -2:]
        gaps = (top2[:, 1] - top2[:, 0]).tolist()
    off = wk["line_off"]
    same = sum(1 for b, r in enumerate(ref["seqs"])
               if np.array_equal(r, gpu["seq"][off[b]:off[b] + gpu["seq_len"][b]]))
    return {"rows": int(ref["idx"].size), "argmax_mismatches": int(mis.size),
            "max_top2_gap_of_mismatches": max(gaps) if gaps else None,
            "maxprob_max_abs_diff": float(np.abs(ref["maxprob"] - gpu["maxprob"]).max()),
            "lines": len(ref["seqs"]), "ctc_sequences_identical": same,
            "score_max_abs_diff": float(np.abs(ref["score"] - gpu["score"]).max())}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def fp32_accuracy(samples):
    """Config fp32_64's variants against the oracle (the C restatement of the reference's
    FP32 matmul_transposed_b, src/ops/matmul.rs:514-897) on the sampled rows their logits
    were kept for: max |GPU logit - oracle logit|."""
    from oracle import oracle as orc
    out = {}
    for variant, (rows, a, w_t, bias, got) in samples.items():
        ref = orc.matmul_transposed_b(a[rows], w_t, bias)
        out[variant] = {"logits_max_abs_vs_oracle": float(np.abs(got - ref).max()), "rows_checked": int(rows.size)}
    return out


def lines_desc(off):
    """'256 lines x T=120', or '29 lines, T=20..120' for lines of several lengths."""
    t = np.diff(np.asarray(off, np.int64))
    if t.size and t.min() == t.max():
        return f"{t.size} lines x T={int(t[0])}"
    return f"{t.size} lines, T={int(t.min()) if t.size else 0}..{int(t.max()) if t.size else 0}"


def cpu_baseline(wk, q, s, seconds, gpu=None):
    """The oracle's line-parallel head (one line per worker, inner serial, as
    src/pipeline.rs:417-433): whole passes over the same batch, repeated to about
    `seconds` of CPU work (one calibration pass first, whose results are also compared
    with the GPU step's when `gpu` holds them)."""
    from oracle import oracle as orc
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    off = wk["line_off"]
    a = wk["a"]
    lines = len(off) - 1
    rows = int(off[-1])
    t0 = time.perf_counter()
    ref = orc.rechead_lines(a, off, q, s, wk["bias"], exec_threads=threads)
    t_pass = time.perf_counter() - t0
    passes = max(1, int(round(seconds / max(t_pass, 1e-6))))
    t0 = time.perf_counter()
    for _ in range(passes):
        orc.rechead_lines(a, off, q, s, wk["bias"], exec_threads=threads)
    dt = time.perf_counter() - t0
    out = {"value": round(passes * rows / dt, 1), "unit": "rows/s", "cores": threads, "kind": "port",
           "cpu_model": cpu_model(),
           "sample": f"{passes} passes over the batch ({lines_desc(off)} = {rows} rows each, "
                     f"{passes * rows} rows), INT8 AVX2 path of the reference restated in C, one line per "
                     f"OpenMP thread, {dt:.1f} s"}
    if gpu is not None:
        out["agreement_with_gpu_step"] = agreement(wk, q, s, ref, gpu)
    return out


def copy_probe(mib):
    """A device-to-device copy of a known size, timed with HIP events: the calibration
    run for the HBM byte counters (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of the copy
    kernel against its known bytes)."""
    from ppocr_rechead.hip import D2D, DeviceArray, Event, check, hip, synchronize
    import ctypes
    nbytes = mib << 20
    src = DeviceArray((nbytes,), np.uint8)
    dst = DeviceArray((nbytes,), np.uint8)
    src.fill_bytes(1)
    synchronize()
    e0, e1 = Event(), Event()
    e0.record(None)
    check(hip().hipMemcpy(dst.p, src.p, ctypes.c_size_t(nbytes), D2D), "hipMemcpy D2D")
    e1.record(None)
    e1.synchronize()
    ms = e0.elapsed_ms(e1)
    src.free()
    dst.free()
    return {"bytes_read": nbytes, "bytes_written": nbytes, "ms": round(ms, 4),
            "GBps_read_plus_write": round(2 * nbytes / (ms / 1e3) / 1e9, 1)}


def write_probe(nbytes):
    """HBM write ceiling: streaming 16-byte stores over a buffer of `nbytes` (the probe
    library's write kernel, timed with HIP events): the bound of the unfused logits writer,
    which stores the same bytes."""
    import ctypes
    from ppocr_rechead.hip import DeviceArray, synchronize
    lib = ctypes.CDLL(os.path.join(ROOT, "rust-ppocrv6_amd", "lib", "libppocr_probe.so"))
    nbytes -= nbytes % 16
    buf = DeviceArray((nbytes,), np.uint8)
    gb, ms = ctypes.c_double(), ctypes.c_double()
    rc = lib.ppocr_probe_write(buf.p, ctypes.c_int64(nbytes), ctypes.byref(gb), ctypes.byref(ms))
    synchronize()
    buf.free()
    if rc:
        raise RuntimeError(f"write probe failed ({rc})")
    return {"bytes": nbytes, "ms": round(ms.value, 4), "GBps": round(gb.value, 1)}


def measured_peaks(write_bytes=0):
    """Peaks measured on this GPU in the same run, beside the datasheet ones: dense bf16
    MFMA with every operand in registers (the benchmark's probe library), a 256 MiB
    device-to-device copy and, with write_bytes, streaming writes of that many bytes."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "rust-ppocrv6_amd", "lib", "libppocr_probe.so"))
    tf, ms = ctypes.c_double(), ctypes.c_double()
    rc = lib.ppocr_probe_mfma_bf16(ctypes.c_int(20000), ctypes.byref(tf), ctypes.byref(ms))
    if rc:
        raise RuntimeError(f"MFMA peak probe failed ({rc})")
    tfd, msd = ctypes.c_double(), ctypes.c_double()
    rc = lib.ppocr_probe_mfma_bf16_data(ctypes.c_int(10000), ctypes.byref(tfd), ctypes.byref(msd))
    if rc:
        raise RuntimeError(f"MFMA data-operand probe failed ({rc})")
    cp = copy_probe(256)
    out = {"bf16_mfma_TFLOPs": round(tf.value, 1), "mfma_probe_ms": round(ms.value, 3),
           "bf16_mfma_TFLOPs_kernel_operands": round(tfd.value, 1), "mfma_data_probe_ms": round(msd.value, 3),
           "copy_GBps_read_plus_write": cp["GBps_read_plus_write"]}
    if write_bytes:
        wp = write_probe(write_bytes)
        out["stream_write_GBps"] = wp["GBps"]
        out["stream_write_bytes"] = wp["bytes"]
    return out


def neck_kernels(nk, dfx, dsc, m, doff, lines, dfeat, dnws, nws, stream, neck_step, work, reps):
    """Each kernel of the SVTR tail timed on its own: the forward with a HIP event between
    its launches (ppocr_rn_forward_marked_dev), each marked forward queued behind an unmarked
    one so the intervals hold kernels, not launch latency; averaged over `reps` forwards.
    Each kernel is set against its binding bound: the fp16 MFMA rate measured on the tail's
    operand patterns divided by the 3 products of the fp16-halves arithmetic (algorithmic
    flops), or the HBM rate of a device copy (algorithmic bytes), whichever takes longer."""
    import ctypes
    import ppocr_rechead as rh
    from ppocr_rechead.hip import Event
    L = rh._lib.lib()
    plib = ctypes.CDLL(os.path.join(ROOT, "rust-ppocrv6_amd", "lib", "libppocr_probe.so"))
    tf, pms = ctypes.c_double(), ctypes.c_double()
    rc = plib.ppocr_probe_mfma_f16_data(ctypes.c_int(10000), ctypes.byref(tf), ctypes.byref(pms))
    if rc:
        raise RuntimeError(f"fp16 MFMA probe failed ({rc})")
    hbm = copy_probe(256)["GBps_read_plus_write"]
    products = 3 if nk.gemm_halves else None
    ceiling = tf.value / products if products else FP32_PEAK_TFLOPS
    ne = 16
    evs = [Event() for _ in range(ne)]
    ev_arr = (ctypes.c_void_p * ne)(*[e.h.value for e in evs])
    names = (ctypes.c_char_p * ne)()
    rec = ctypes.c_int()
    acc = None
    ramp(neck_step, 0.05)
    for _ in range(reps):
        neck_step()
        rh._check(L.ppocr_rn_forward_marked_dev(nk.handle, dfx.p, dsc.p, m, doff.p, lines, rh.NECK_ROWS, dfeat.p,
                                                dnws.p, nws, stream.h, ev_arr, ne, names, ctypes.byref(rec)))
        evs[rec.value - 1].synchronize()
        t = [evs[i - 1].elapsed_ms(evs[i]) for i in range(1, rec.value)]
        acc = t if acc is None else [x + y for x, y in zip(acc, t)]
    got = [names[i].decode() for i in range(1, rec.value)]
    if got != [w[0] for w in work]:
        raise RuntimeError(f"tail kernels {got} do not match the work model {[w[0] for w in work]}")
    out = []
    for (name, flops, nbytes), tot in zip(work, acc):
        ms = tot / reps
        t_m = flops / (ceiling * 1e12) * 1e3
        t_h = nbytes / (hbm * 1e9) * 1e3
        out.append({"name": name, "ms": round(ms, 4), "GFLOP": round(flops / 1e9, 3), "MB": round(nbytes / 1e6, 2),
                    "TFLOPs": round(flops / (ms / 1e3) / 1e12, 1), "GBps": round(nbytes / (ms / 1e3) / 1e9, 1),
                    "bound": "mfma" if t_m >= t_h else "hbm", "bound_ms": round(max(t_m, t_h), 4),
                    "frac": round(max(t_m, t_h) / ms, 4)})
    bound = {"f16_mfma_TFLOPs_tail_operands": round(tf.value, 1), "products_per_multiply_add": products,
             "mfma_ceiling_TFLOPs": round(ceiling, 1), "copy_GBps_read_plus_write": hbm,
             "marked_forward_ms": round(sum(acc) / reps, 4)}
    return out, bound


def make_workload(name):
    """A workload by name; the stress batch packs its weights with the GPU packer first
    (its near-tie rows are placed on the dequantised weights)."""
    import ppocr_rechead as rh
    from ppocr_rechead import workloads as wl

    def pack(w_t):
        qw = rh.QuantizedWeight.from_f32_transposed(w_t)
        return qw.data, qw.scales

    return wl.make(name, pack=pack if name == "stress_1024" else None)


def other_config(name, modes, steps, warmup, samples=None):
    """Fused decode step (argmax + CTC) of another configuration, per mode; for an FP32
    head also the logits kernel alone (the unfused projection), whose logits of a row
    sample (the first and last 128 rows and 256 seeded others) go to `samples` for the
    accuracy check; for a head whose mode has a precision guard, the rows over it."""
    import ppocr_rechead as rh
    from ppocr_rechead import workloads as wl
    from ppocr_rechead.hip import DeviceArray, Stream
    L = rh._lib.lib()
    wk = make_workload(name)
    a = wk["a"]
    m, k = a.shape
    n = wl.N_CLASSES
    lines = len(wk["line_off"]) - 1
    if wk["quantized"]:
        qw = (rh.QuantizedWeight(wk["q"], wk["scales"]) if "q" in wk
              else rh.QuantizedWeight.from_f32_transposed(wk["w_t"]))
        head = rh.RecHead(qw=qw, bias=wk["bias"])
    else:
        head = rh.RecHead(w_t=wk["w_t"], bias=wk["bias"])
    stream = Stream()
    st = stream.h
    da = DeviceArray.from_numpy(a)
    doff = DeviceArray.from_numpy(wk["line_off"])
    didx, dmp, dseq = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32), DeviceArray((m,), np.int32)
    dlen, dscore = DeviceArray((lines,), np.int64), DeviceArray((lines,), np.float32)
    res = {"rows": m, "lines": lines, "head": "int8" if wk["quantized"] else "fp32",
           "auto_mode": MODE_NAMES[head.auto_mode()]}
    for mode in modes:
        ws = head.workspace_bytes(m, mode)
        dws = DeviceArray((max(ws, 1),), np.uint8)

        def step():
            rh._check(L.ppocr_rh_decode_dev(head.handle, da.p, m, doff.p, lines, mode, didx.p, dmp.p, dseq.p,
                                            dlen.p, dscore.p, dws.p, ws, st))

        ramp(step)
        ms, _ = timed(step, stream, steps, warmup)
        flops = 2.0 * m * n * k
        r = {"ms_per_step": round(ms, 4), "rows_per_s": round(m / (ms / 1e3), 1),
             "TFLOPs": round(flops / (ms / 1e3) / 1e12, 2)}
        prec, ra, rn = head.guard_limits(mode)
        if np.isfinite(prec):
            r["guarded_rows"] = int(head.guarded_rows(a, mode).sum())
            r["guard_limits"] = {"precision_max_abs": round(prec, 4), "range_max_abs": round(ra, 4),
                                 "range_norm": round(rn, 4)}
        if wk["quantized"] and m <= 8192:
            # the same step from host arrays (ppocr_rh_decode): what one call per page costs
            off = wk["line_off"]
            for _ in range(3):
                head.decode(a, off, mode)
            t0 = time.perf_counter()
            for _ in range(steps):
                head.decode(a, off, mode)
            r["host_arrays_ms"] = round((time.perf_counter() - t0) / steps * 1e3, 4)
        if not wk["quantized"]:
            dlog = DeviceArray((m, n), np.float32)

            def logits():
                rh._check(L.ppocr_rh_logits_dev(head.handle, da.p, m, mode, dlog.p, dws.p, ws, st))

            ms_l, _ = timed(logits, stream, max(3, steps // 2), 2)
            lb = 4.0 * m * n + 4.0 * m * k + 4.0 * n * k + 4.0 * n
            r["logits_ms"] = round(ms_l, 4)
            r["logits_GBps"] = round(lb / (ms_l / 1e3) / 1e9, 1)
            if samples is not None:
                rng = np.random.default_rng(0x5EED0200)
                rows = np.unique(np.concatenate([np.arange(min(128, m)), np.arange(max(0, m - 128), m),
                                                 rng.integers(0, m, 256)]))
                samples["fp32_fma" if mode == 0 else MODE_NAMES[mode]] = (rows, a, wk["w_t"], wk["bias"],
                                                                          dlog.numpy()[rows])
            dlog.free()
        res["fp32_fma" if mode == 0 else MODE_NAMES[mode]] = r
        dws.free()
    head.close()
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU: the head shards along rows with the "
                                   "weights replicated, so more GPUs are not measured here"}))
        sys.exit(2)

    import ppocr_rechead as rh
    from ppocr_rechead import workloads as wl
    from ppocr_rechead.hip import DeviceArray, Stream, synchronize

    L = rh._lib.lib()
    wk = make_workload(args.workload)
    a = wk["a"]
    m, k = a.shape
    n = wl.N_CLASSES
    lines = len(wk["line_off"]) - 1
    qw = rh.QuantizedWeight.from_f32_transposed(wk["w_t"])  # GPU packer
    head = rh.RecHead(qw=qw, bias=wk["bias"])
    mode = args.mode
    rmode = head.auto_mode() if mode == 5 else mode  # the arithmetic the mode runs on this head

    stream = Stream()
    st = stream.h
    da = DeviceArray.from_numpy(a)
    doff = DeviceArray.from_numpy(wk["line_off"])
    didx = DeviceArray((m,), np.int32)
    dmp = DeviceArray((m,), np.float32)
    dseq = DeviceArray((m,), np.int32)
    dlen = DeviceArray((lines,), np.int64)
    dscore = DeviceArray((lines,), np.float32)
    ws_bytes = head.workspace_bytes(m, mode)
    dws = DeviceArray((max(ws_bytes, 1),), np.uint8)
    synchronize()

    def fused_argmax():
        rh._check(L.ppocr_rh_argmax_dev(head.handle, da.p, m, mode, didx.p, dmp.p, dws.p, ws_bytes, st))

    def ctc():
        rh._check(L.ppocr_ctc_greedy_dev(didx.p, dmp.p, doff.p, lines, 0, dseq.p, dlen.p, dscore.p, st))

    def fused_step():
        # the whole head as one call: projection + softmax statistics, then the chunk merge
        # and the CTC collapse in one kernel
        rh._check(L.ppocr_rh_decode_dev(head.handle, da.p, m, doff.p, lines, mode, didx.p, dmp.p, dseq.p, dlen.p,
                                        dscore.p, dws.p, ws_bytes, st))

    out = {}
    flops = 2.0 * m * n * k
    if args.only in ("", "fused"):
        ramp(fused_step)
        ms_step, wall_ms = timed(fused_step, stream, args.steps, args.warmup)
        synchronize()
        gpu_res = {"idx": didx.numpy(), "maxprob": dmp.numpy(), "seq": dseq.numpy(), "seq_len": dlen.numpy(),
                   "score": dscore.numpy()}
        ms_head, _ = timed(fused_argmax, stream, args.steps, args.warmup)
        out["fused"] = (ms_step, wall_ms, ms_head)
        # the library's default arithmetic (AUTO: the mode the head's weights suit) on the
        # same batch, beside the split the headline runs
        default = None
        if mode != 5:
            aws = head.workspace_bytes(m, 5)
            daws = DeviceArray((max(aws, 1),), np.uint8)

            def auto_step():
                rh._check(L.ppocr_rh_decode_dev(head.handle, da.p, m, doff.p, lines, 5, didx.p, dmp.p, dseq.p,
                                                dlen.p, dscore.p, daws.p, aws, st))

            ramp(auto_step, 0.05)
            ms_auto, _ = timed(auto_step, stream, args.steps, args.warmup)
            amode = head.auto_mode()
            default = {"mode": f"auto ({MODE_NAMES[amode]})", "ms_per_step": round(ms_auto, 5),
                       "rows_per_s": round(m / (ms_auto / 1e3), 1),
                       "guarded_rows": int(head.guarded_rows(a, amode).sum()) if amode in TERMS else 0}
            daws.free()
        out["default"] = default

    unf = None
    if args.only in ("", "unfused"):
        dlog = DeviceArray((m, n), np.float32)

        def unfused_step():
            rh._check(L.ppocr_rh_logits_dev(head.handle, da.p, m, mode, dlog.p, dws.p, ws_bytes, st))
            rh._check(L.ppocr_softmax_rows_dev(dlog.p, m, n, didx.p, dmp.p, st))
            ctc()

        def logits_only():
            rh._check(L.ppocr_rh_logits_dev(head.handle, da.p, m, mode, dlog.p, dws.p, ws_bytes, st))

        ms_u, _ = timed(unfused_step, stream, max(3, args.steps // 2), 2)
        ms_l, _ = timed(logits_only, stream, max(3, args.steps // 2), 2)
        logits_bytes = 4.0 * m * n + 4.0 * m * k + 1.0 * n * k + 8.0 * n
        total_bytes = logits_bytes + 8.0 * m * n + 8.0 * m
        unf = {"ms_per_step": round(ms_u, 4), "rows_per_s": round(m / (ms_u / 1e3), 1),
               "algorithmic_GBps": round(total_bytes / (ms_u / 1e3) / 1e9, 1),
               "logits_kernel_ms": round(ms_l, 4),
               "logits_kernel_GBps": round(logits_bytes / (ms_l / 1e3) / 1e9, 1),
               "logits_hbm_frac": round(logits_bytes / (ms_l / 1e3) / 1e9 / HBM_PEAK_GBS, 4)}
        dlog.free()

    neck = None
    if args.only in ("", "neck"):
        # the SVTR tail before the head on the same lines (synthetic weights of the real
        # model's statistics), alone and followed by the fused head: the head's input then
        # never leaves the device
        nw = wl.neck_weights()
        nk = rh.RecNeck(nw["blocks"], nw["lnf_w"], nw["lnf_b"], nw["lnf_eps"])
        rng = np.random.default_rng(wl.SEED_A + 0x77)
        dfx = DeviceArray.from_numpy((rng.standard_normal((m, k)) * 1.5).astype(np.float32))
        dsc = DeviceArray.from_numpy(rng.standard_normal((m, k)).astype(np.float32))
        dfeat = DeviceArray((m, k), np.float32)
        nws = nk.workspace_bytes(m)
        dnws = DeviceArray((nws,), np.uint8)

        def neck_step():
            rh._check(L.ppocr_rn_forward_dev(nk.handle, dfx.p, dsc.p, m, doff.p, lines, rh.NECK_ROWS, dfeat.p,
                                             dnws.p, nws, st))

        ramp(neck_step)
        ms_n, _ = timed(neck_step, stream, args.steps, args.warmup)
        steps_of = np.diff(wk["line_off"])
        nflops = float(sum(int(t) * wl.neck_flops_per_row(int(t)) for t in steps_of))
        synchronize()
        feats = dfeat.numpy()
        kernels, bound = neck_kernels(nk, dfx, dsc, m, doff, lines, dfeat, dnws, nws, stream, neck_step,
                                      wl.neck_kernel_work(steps_of, len(nw["blocks"])), max(20, args.steps // 4))
        neck = {"blocks": len(nw["blocks"]), "ms_per_step": round(ms_n, 4), "rows_per_s": round(m / (ms_n / 1e3), 1),
                "TFLOPs": round(nflops / (ms_n / 1e3) / 1e12, 2),
                "flops_per_step": nflops, "head_input_max_abs": round(float(np.abs(feats).max()), 2),
                "matmul_arithmetic": "fp16 halves (3 products)" if nk.gemm_halves else "fp32",
                "bound": bound, "kernels": kernels,
                "frac_of_binding_bound": round(sum(x["bound_ms"] for x in kernels) / ms_n, 4),
                "neck_then_head": {}}
        for hm in sorted({mode, 5}):
            hws = head.workspace_bytes(m, hm)
            dhws = DeviceArray((max(hws, 1),), np.uint8)

            def neck_head_step():
                neck_step()
                rh._check(L.ppocr_rh_decode_dev(head.handle, dfeat.p, m, doff.p, lines, hm, didx.p, dmp.p, dseq.p,
                                                dlen.p, dscore.p, dhws.p, hws, st))

            ramp(neck_head_step)
            ms_nh, _ = timed(neck_head_step, stream, args.steps, args.warmup)
            rm = head.auto_mode() if hm == 5 else hm
            neck["neck_then_head"][MODE_NAMES[hm] + (f" ({MODE_NAMES[rm]})" if hm == 5 else "")] = {
                "ms_per_step": round(ms_nh, 4), "rows_per_s": round(m / (ms_nh / 1e3), 1),
                "guarded_rows": int(head.guarded_rows(feats, rm).sum()) if rm in (2, 3, 4) else 0}
            dhws.free()
        for d in (dfx, dsc, dfeat, dnws):
            d.free()
        nk.close()

    probs = None
    if args.only in ("", "probs"):
        dprobs = DeviceArray((m, n), np.float32)
        pws = head.workspace_bytes(m, mode)

        def probs_step():
            rh._check(L.ppocr_rh_probs_dev(head.handle, da.p, m, mode, dprobs.p, dws.p, pws, st))

        ms_p, _ = timed(probs_step, stream, max(3, args.steps // 2), 2)
        pbytes = 4.0 * m * n
        probs = {"ms_per_step": round(ms_p, 4), "rows_per_s": round(m / (ms_p / 1e3), 1),
                 "probs_write_GBps": round(pbytes / (ms_p / 1e3) / 1e9, 1),
                 "hbm_frac": round(pbytes / (ms_p / 1e3) / 1e9 / HBM_PEAK_GBS, 4)}
        dprobs.free()

    host = None
    if args.only == "":
        # the same step from host arrays to host results (ppocr_rh_decode: PCIe both ways);
        # reported beside the device rate, never as `value`
        off = wk["line_off"]
        for _ in range(2):
            head.decode(a, off, mode)
        reps = max(3, args.steps // 2)
        t0 = time.perf_counter()
        for _ in range(reps):
            head.decode(a, off, mode)
        host_ms = (time.perf_counter() - t0) / reps * 1e3
        host = {"ms_per_step": round(host_ms, 4), "rows_per_s": round(m / (host_ms / 1e3), 1),
                "entry": "ppocr_rh_decode (host activations in, host sequences out)"}

    copy = copy_probe(args.copy_probe) if args.copy_probe > 0 else None
    peaks = measured_peaks(int(4 * m * n)) if args.only == "" else None
    if unf and peaks and peaks.get("stream_write_GBps"):
        # the logits writer against the streaming-write ceiling of the same bytes
        unf["stream_write_GBps"] = peaks["stream_write_GBps"]
        unf["logits_frac_of_stream_write"] = round(unf["logits_kernel_GBps"] / peaks["stream_write_GBps"], 4)

    others = None
    fp32_samples = {}
    if args.only == "" and not args.no_others:
        others = {"single_line": other_config("single_line", (2, 4), args.steps, args.warmup),
                  "a4_page": other_config("a4_page", (2, 3, 4), args.steps, args.warmup),
                  args.workload: other_config(args.workload, tuple(x for x in (2, 3, 4) if x != rmode),
                                              args.steps, args.warmup),
                  "fp32_64": other_config("fp32_64", (0, 3, 4), args.steps, args.warmup, fp32_samples),
                  "stress_1024": other_config("stress_1024", (2, 4), max(3, args.steps // 4), 2)}

    cpu = None
    if not args.no_cpu and args.only == "":
        cpu = cpu_baseline(wk, qw.data, qw.scales, args.cpu_seconds, gpu_res if "fused" in out else None)
        if fp32_samples:
            for variant, acc in fp32_accuracy(fp32_samples).items():
                others["fp32_64"][variant].update(acc)

    if "fused" in out:
        ms_step, wall_ms, ms_head = out["fused"]
        achieved = flops / (ms_head / 1e3) / 1e12
        peak = FP32_PEAK_TFLOPS if rmode == 0 else BF16_PEAK_TFLOPS
        ceiling = None
        if peaks and rmode in TERMS:
            # t products per logit: at most 1/t of the measured dense MFMA rate is useful work
            t = TERMS[rmode]
            # the second ceiling: the rate the matrix cores hold on operands like the
            # kernel's (the GPU's power limit lowers the clock on such bit patterns)
            dr = peaks["bf16_mfma_TFLOPs_kernel_operands"]
            ceiling = {"terms": t, "measured_mfma_TFLOPs": peaks["bf16_mfma_TFLOPs"],
                       "ceiling_TFLOPs": round(peaks["bf16_mfma_TFLOPs"] / t, 1),
                       "frac_of_ceiling": round(achieved / (peaks["bf16_mfma_TFLOPs"] / t), 4),
                       "kernel_operand_mfma_TFLOPs": dr, "kernel_operand_ceiling_TFLOPs": round(dr / t, 1),
                       "frac_of_kernel_operand_ceiling": round(achieved / (dr / t), 4)}
        line = {
            "metric": "rec-head rows/s (B*T x 18710 INT8 proj+softmax+CTC)",
            "value": round(m / (ms_step / 1e3), 1),
            "unit": "rows/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms_step, 5),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": MODE_NAMES[rmode] + " MFMA, f32 accumulate, int8 weights" if rmode else "f32 FMA, int8 weights",
            "data": "synthetic (seeded N(0,1) activations, N(0,0.05^2) weights packed to INT8 on the GPU)",
            "config": {"workload": f"{args.workload}: {lines_desc(wk['line_off'])}, m={m}, k={k}, n={n}, fused "
                                   "projection+softmax-max+argmax+CTC",
                       "mode": MODE_NAMES[mode] + (f" ({MODE_NAMES[rmode]})" if mode == 5 else ""),
                       "guarded_rows": int(head.guarded_rows(a, rmode).sum()) if rmode in TERMS else 0,
                       "clock_ramp_s": 0.2},
            "library_default": out.get("default"),
            "roofline": {"bound": "mfma" if rmode else "valu",
                         "kernel": "ppocr_rh_argmax_dev: stats_main_kernel (>= 95% of the time) + "
                                   "guarded-row rescue and merge kernels",
                         "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                         "frac": round(achieved / peak, 4), "traffic": traffic_from_profiles("stats_main_kernel_dense_256"),
                         "algorithmic_flops_per_launch": flops, "kernel_ms": round(ms_head, 5),
                         "split_ceiling": ceiling},
            "measured_peaks": peaks,
            "wall_ms_per_step": round(wall_ms, 5),
            "host_arrays": host,
            "unfused": unf,
            "probs_fused": probs,
            "neck": neck,
            "cpu_baseline": cpu,
            "other_configs": others,
        }
        if copy:
            line["copy_probe"] = copy
    else:
        line = {"metric": "profiling run", "unfused": unf, "probs_fused": probs, "neck": neck, "copy_probe": copy}
    print(json.dumps(line), flush=True)
    head.close()


if __name__ == "__main__":
    main()
