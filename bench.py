"""Throughput of the HIP backend on the det + rec workload, one JSON line.

A step is one det forward on 1x3x640x640 plus one rec forward on a batch of
32 lines of 3x48x320 (the det image and the 32 text lines of one page), both
as replayed HIP graphs with their inputs already resident in HBM.  The det
and rec sessions run on two contexts (two streams), as a page pipeline runs
the det of one page next to the rec of another: value = steps per second =
det images per second with 32 recognised lines each, over the wall time of
K steps with both streams busy.  det_img_per_s and rec_lines_per_s are the
stage-isolated rates (HIP events around each session alone, on its own
stream) and serial_ms_per_step their sum, the step time on one stream.

roofline: the dominant kernel is the rec head GEMM (1280 x 18709 x 256,
12.26 GFLOP of the step's 20.86).  Its average launch time comes from HIP
events around each node of the rec graph (eager launches on the same stream),
over the same number of steps, after the timed region.  traffic (HBM bytes
per launch) is the calibrated FETCH_SIZE + WRITE_SIZE figure recorded in
profiles/rec_head_gemm_traffic.md (rocprofv3 counter runs of this script).

cpu_baseline: the CPU oracle (plain-C restatement of the qppocr-kernels
AVX2 path, OpenMP over all host threads) on a bounded sample of the same
workload, timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
REC_BATCH = 32


def head_traffic_bytes():
    """HBM bytes per launch of the rec head GEMM from the committed counter
    summary, or None when it is absent."""
    path = os.path.join(ROOT, "profiles", "rec_head_gemm_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch"):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


OP_NAMES = {1: "conv", 2: "convt_pair_sigmoid", 3: "linear", 4: "layernorm", 5: "attention",
            6: "softmax_argmax", 7: "convt", 8: "act"}


def write_node_report(path, nets, graphs):
    """Per node: average launch time (HIP events, eager launches) and the
    fraction of its roofline (fp32 MFMA peak for products, HBM peak else)."""
    rows = []
    for name, g, node_ms in graphs:
        for i, d in enumerate(g.nodes):
            fl, by, bound = nets.node_cost(g, d)
            ms = node_ms[i]
            row = {"graph": name, "node": i, "op": OP_NAMES.get(d["op"], str(d["op"])),
                   "in": list(g.lshapes[d["inp"]]), "w": list(d["ws"]), "us": round(ms * 1e3, 2),
                   "gflop": round(fl / 1e9, 4), "mb": round(by / 1e6, 3), "bound": bound}
            if ms > 0:
                tf, gbs = fl / (ms * 1e-3) / 1e12, by / (ms * 1e-3) / 1e9
                row["tflops"], row["gbs"] = round(tf, 2), round(gbs, 1)
                row["frac"] = round(tf / PEAK_FP32_MFMA_TFLOPS if bound == "mfma"
                                    else gbs / PEAK_HBM_GBS, 4)
            rows.append(row)
    with open(path, "w") as f:
        json.dump(rows, f, indent=0)


def time_mixed_page(steps, warmup):
    """det 1x3x1536x1536 + 128 rec lines (widths {80..1280}, buckets of 160,
    <= 64 lines per batch), inputs resident.  det and the rec batches run on
    three streams (det; rec batches alternating over two): page_ms is the
    wall time per page over the steps; det_ms / rec_ms are each stage alone."""
    import torch
    from qppocr_amd import ops, pipeline
    det_g, det_x, rw, lines, widths = pipeline.mixed_page(4, 1536, 128)
    ctxs = [ops.new_context(0) for _ in range(3)]
    page = pipeline.PageRunner(det_g, det_x, rw, lines, widths, contexts=ctxs)
    page.upload()
    for _ in range(warmup):
        page.run()
    page.sync()

    def wall(fn):
        page.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        page.sync()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps
    det_ms = wall(page.run_det)
    rec_ms = wall(page.run_rec)
    page_ms = wall(page.run)
    out = {"workload": "det 1x3x1536x1536 + 128 rec lines 3x48x{80..1280}, buckets of 160, "
                       "<= 64 lines/batch, CTC masked past w/8",
           "rec_batches": [[bw, len(idx)] for bw, idx in page.plan],
           "det_img_per_s": round(1e3 / det_ms, 2),
           "rec_lines_per_s": round(len(widths) * 1e3 / rec_ms, 1),
           "page_ms": round(page_ms, 4), "det_ms": round(det_ms, 4),
           "rec_ms": round(rec_ms, 4)}
    page.close()
    for c in ctxs:
        ops.close_context(c)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-steps", type=int, default=6, help="CPU baseline sample (steps)")
    ap.add_argument("--mixed-page", action="store_true",
                    help="also time the mixed-shape page (det 1536^2 + 128 bucketed rec lines)")
    ap.add_argument("--node-report", default="",
                    help="also write per-node times and roofline fractions (JSON) to this path")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (a kernel of "
                         "known traffic for scaling FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only; the det/rec path "
                          "shards by image / rec batch with no exchange between GPUs, "
                          "and multi-GPU runs are not part of it", "n_gpus": args.gpus}))
        sys.exit(2)

    import numpy as np
    import torch
    from qppocr_amd import nets, ops

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    ctx = ops.context(0)           # det stream
    ctx_rec = ops.new_context(0)   # rec stream
    lib = ops._lib.load()
    stream = torch.cuda.ExternalStream(lib.qph_ctx_stream(ctx))
    stream_rec = torch.cuda.ExternalStream(lib.qph_ctx_stream(ctx_rec))
    if args.copy_calibration_mb > 0:
        n = args.copy_calibration_mb * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    det_g, det_x = nets.build_det(2, 640, 640)
    rec_g, rec_x = nets.build_rec(3, REC_BATCH, 320)
    det = nets.HipSession(det_g, ctx=ctx)
    rec = nets.HipSession(rec_g, ctx=ctx_rec)
    # inputs resident in HBM: copied once, then every step reuses them
    det.run(det_x, outputs=False)
    rec.run(rec_x, outputs=False)
    det.sync()
    rec.sync()

    def both_sync():
        det.sync()
        rec.sync()
        torch.cuda.synchronize()

    for _ in range(args.warmup):
        det.run(None, outputs=False)
        rec.run(None, outputs=False)
    both_sync()

    K = args.steps
    # stage-isolated times: each session alone on its own stream
    def stage_ms(sess, st):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(K):
            sess.run(None, outputs=False)
        e1.record(st)
        both_sync()
        return e0.elapsed_time(e1) / K
    det_ms = stage_ms(det, stream)
    rec_ms = stage_ms(rec, stream_rec)

    # the timed region: K steps, det and rec of each step on their streams
    both_sync()
    t0 = time.perf_counter()
    for i in range(K):
        det.run(None, outputs=False)
        rec.run(None, outputs=False)
    both_sync()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / K

    # the same step with host buffers at the boundary: det input up, det map
    # down, rec input up, rec (val, idx) pairs down (pageable host memory)
    pairs_id = rec_g.outputs[-1]
    pairs_ptr, pairs_n = rec.tensor_ptr(pairs_id)
    pairs_host = np.empty(pairs_n, np.float32)
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    for _ in range(K):
        det.run(det_x, outputs=True)
        rec.run(rec_x, outputs=False)
        ops.check(lib.qph_memcpy_d2h(ctx_rec, pairs_host.ctypes.data_as(ctypes.c_void_p),
                                     ctypes.c_void_p(pairs_ptr), pairs_n * 4))
    both_sync()
    h1 = time.perf_counter()
    host_ms_step = (h1 - h0) * 1e3 / K

    # dominant kernel: rec head GEMM, events around each node (eager launches)
    rec.set_profiling(True)
    for _ in range(K):
        rec.run(None, outputs=False)
    rec.sync()
    node_ms = rec.node_times()
    rec.set_profiling(False)
    head = len(rec_g.nodes) - 2        # linear 256 -> 18709
    head_ms = node_ms[head]
    d = rec_g.nodes[head]
    rows = rec_g.numel(d["inp"]) // d["ws"][0]
    head_flops = 2 * rows * d["ws"][0] * d["ws"][1]
    achieved = head_flops / (head_ms * 1e-3) / 1e12

    if args.node_report:
        det.set_profiling(True)
        for _ in range(K):
            det.run(None, outputs=False)
        det.sync()
        det_node_ms = det.node_times()
        det.set_profiling(False)
        write_node_report(args.node_report, nets, [("det", det_g, det_node_ms),
                                                   ("rec", rec_g, node_ms)])

    det_flops = nets.flops(det_g)
    rec_flops = nets.flops(rec_g)
    result = {
        "metric": "det img/s @1x3x640x640 + rec lines/s @48x320 b32, fp32; % of roofline",
        "value": round(1e3 / ms_step, 3),
        "unit": "img/s (1 det image 1x3x640x640 + 32 rec lines 3x48x320 per step)",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded inputs, random-init weights)",
        "config": {"workload": "det 1x3x640x640 (config 3) + rec 32x3x48x320 (config 4) per step",
                   "det_gflop": round(det_flops / 1e9, 3), "rec_gflop": round(rec_flops / 1e9, 3)},
        "det_img_per_s": round(1e3 / det_ms, 2),
        "rec_lines_per_s": round(REC_BATCH * 1e3 / rec_ms, 1),
        "det_ms": round(det_ms, 4),
        "rec_ms": round(rec_ms, 4),
        "serial_ms_per_step": round(det_ms + rec_ms, 4),
        "pcie_inclusive_img_per_s": round(1e3 / host_ms_step, 3),
        "roofline": {"bound": "mfma", "kernel": "rec head GEMM 1280x18709x256 (gemm_wave_kernel)",
                     "achieved": round(achieved, 2), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
                     "traffic": head_traffic_bytes(), "avg_launch_ms": round(head_ms, 5)},
    }

    if args.mixed_page:
        result["mixed_page"] = time_mixed_page(K, args.warmup)

    if not args.no_cpu:
        from oracle import nets as onets
        from oracle import oracle as O
        O.lib()
        onets.run_graph(det_g, det_x)          # warm-up (page-in, thread pool)
        c0 = time.perf_counter()
        for _ in range(args.cpu_steps):
            onets.run_graph(det_g, det_x)
            onets.run_graph(rec_g, rec_x)
        c1 = time.perf_counter()
        cpu_step = (c1 - c0) / args.cpu_steps
        result["cpu_baseline"] = {
            "value": round(1.0 / cpu_step, 4),
            "unit": result["unit"],
            "cores": O.threads(),
            "kind": "port",
            "sample": f"{args.cpu_steps} steps of det 1x3x640x640 + rec 32x3x48x320, "
                      f"{cpu_step:.3f} s/step, C oracle -O3 -mavx2 -mfma, OpenMP",
        }
    print(json.dumps(result))
    det.close()
    rec.close()
    ops.close_context(ctx_rec)


if __name__ == "__main__":
    main()
