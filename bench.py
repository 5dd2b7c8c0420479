"""Throughput of the HIP backend on the det + rec workload, one JSON line,
with every synthetic config measured beside it.

Headline step: one det forward on 1x3x640x640 plus one rec forward on a
batch of 32 lines of 3x48x320 (the det image and the 32 text lines of one
page), both as replayed HIP graphs with their inputs already resident in
HBM.  The rec session ends in the CTC exit of the reference's GPU sessions
(rec_argmax_pairs, qppocr-core/src/device.rs:160-165): the (value, index)
pairs the decoder reads.  In the headline graph the head linear carries the
softmax + argmax in its epilogue (the fused head: logits never reach HBM;
values within 1e-4 relative of the reference, ids equal except where a
step's top-2 logit gap is below 1e-4).  Beside it: rec_lines_per_s_bitexact_
pairs, the graph with the separate head softmax whose pairs are bit-exact,
and rec_lines_per_s_with_probs, that graph exporting the probability tensor
too.
The det and rec sessions run on contexts (streams) of their own, as a page
pipeline runs the det of one page next to the rec of another, with
--pages-in-flight pages (default 2) in flight at once: page i of the K timed
steps runs on det and rec session pair i % P, each pair on two streams of
its own (2 pages: 4 streams, the hardware queues a process gets here).
value = steps per second = det images per second with 32 recognised lines
each, over the wall time of the K steps; one_page_in_flight gives the same K
steps on one det and one rec stream.  det_img_per_s and rec_lines_per_s are
the stage-isolated rates (HIP events around each session alone, on its own
stream).  Defaults: K = 200 timed steps (about 60 ms) after W = 20 warm-up
steps; the per-config, cls and aux legs take their repetitions from
min(K, 50).

roofline: the dominant kernel, the fused rec head (GEMM 1280 x 18709 x
256, 12.26 GFLOP of the step's 20.86, with the softmax / argmax epilogue),
bound by the MFMA pipe.  Its average launch time comes from HIP events
around each node of the rec graph (eager launches on the session stream)
over the same number of steps.  traffic (HBM bytes per launch) is the
calibrated FETCH_SIZE + WRITE_SIZE figure in
profiles/rec_fused_head_traffic.md.  head_gemm_unfused gives the same
figures for the plain head GEMM of the bit-exact graph.

plan_model: the same det and rec graphs lowered to the reference's plan
model (GraphPlan dispatch lists over an NHWC arena) and run by the HIP
kernel set of its n_* dispatch contracts (qph_plan_*), each plan alone.

configs: the five benchmark workloads, each with its GPU rate, the roofline
fraction of its bound and the CPU oracle timed on this host (threads set
explicitly, one warm-up round, then the median of at least --cpu-rounds
rounds, run until each leg has taken 2 s, 5 s for the headline's det and rec):
  cfg1 conv3x3 32->32 @160^2 + bias + ReLU and cfg2a-d depthwise + hardswish:
    the op as a session node with resident weights, replicated over enough
    input/output buffer sets that the sets together exceed 512 MB (twice the
    256 MB Infinity Cache); a graph replay runs the copies back to back, each
    on the next set, so every launch reads its operands cache-cold.  The
    time per launch is the replay's HIP-event time over the copies.
  cfg3 det 640^2 / cfg4 rec 32x320: the headline's stage rates, with the
    per-kernel-class roofline fractions from per-node event times.
  cfg5: det 1536^2 + 128 rec lines in width buckets (page wall time).
  cls (beside the five): the orientation classifier on a full batch of 32
    lines of 3x48x192 (graph replays), lines/s.

aux: the operators around the nets -- page resize, det input normalisation,
rec line packing, the DB mask, the SE block's pool and gate, MaxPool,
bilinear Resize, Transpose -- each at a page-scale shape: device time per
launch, cache-cold (a captured graph over rotating buffer sets past 512 MB),
against the HBM roofline, with the CPU oracle on the same inputs beside each
(1 s floor per operator).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--cpu-rounds R] [--no-configs] [--node-report FILE]
                       [--no-plan] [--plan-only] [--aux-only]
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
REC_BATCH = 32
COLD_BYTES = 512 << 20      # buffer sets per op bench: twice the Infinity Cache
CPU_HEADLINE_MIN_S = 5.0    # CPU oracle: seconds of timed rounds for det and for rec
CPU_CONFIG_MIN_S = 2.0      # ... and for each single-op / page config
CPU_AUX_MIN_S = 1.0         # ... and for each operator of the aux leg


def head_traffic_bytes(name="rec_fused_head_traffic.md"):
    """HBM bytes per launch of a rec head kernel from its committed counter
    summary, or None when it is absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch"):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


OP_NAMES = {1: "conv", 2: "convt_pair_sigmoid", 3: "linear", 4: "layernorm", 5: "attention",
            6: "softmax_argmax", 7: "convt", 8: "act"}


def node_rows(nets, name, g, node_ms):
    rows = []
    for i, d in enumerate(g.nodes):
        fl, by, bound = nets.node_cost(g, d)
        ms = node_ms[i]
        row = {"graph": name, "node": i, "op": OP_NAMES.get(d["op"], str(d["op"])),
               "in": list(g.lshapes[d["inp"]]), "w": list(d["ws"]), "us": round(ms * 1e3, 2),
               "gflop": round(fl / 1e9, 4), "mb": round(by / 1e6, 3), "bound": bound,
               # tensor ids and the bytes "mb" books for them (the input read
               # once, the output written y_up^2 times), so a launch covering
               # several nodes can drop a tensor that never leaves it
               "t_in": d["inp"], "t_out": d["out"],
               "in_mb": round(g.numel(d["inp"]) * 4 / 1e6, 3),
               "out_mb": round(g.numel(d["out"]) * d["y_up"] ** 2 * 4 / 1e6, 3)}
        if ms > 0:
            tf, gbs = fl / (ms * 1e-3) / 1e12, by / (ms * 1e-3) / 1e9
            row["tflops"], row["gbs"] = round(tf, 2), round(gbs, 1)
            row["frac"] = round(tf / PEAK_FP32_MFMA_TFLOPS if bound == "mfma"
                                else gbs / PEAK_HBM_GBS, 4)
        rows.append(row)
    return rows


def class_fractions(nets, g, node_ms):
    """Per roofline class: summed algorithmic work over summed node time
    (eager launches, one event pair per node: an upper bound on the time,
    so a lower bound on the fraction).  Fused launches book their time on
    their first node and 0 on the others; the work of every node counts."""
    agg = {"mfma": [0.0, 0.0], "hbm": [0.0, 0.0]}
    for i, d in enumerate(g.nodes):
        fl, by, bound = nets.node_cost(g, d)
        a = agg[bound]
        a[0] += fl if bound == "mfma" else by
        a[1] += node_ms[i]
    out = {}
    for k, (work, ms) in agg.items():
        if ms <= 0:
            continue
        if k == "mfma":
            tf = work / (ms * 1e-3) / 1e12
            out[k] = {"tflops": round(tf, 2), "frac": round(tf / PEAK_FP32_MFMA_TFLOPS, 4),
                      "us": round(ms * 1e3, 1)}
        else:
            gbs = work / (ms * 1e-3) / 1e9
            out[k] = {"gbs": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
                      "us": round(ms * 1e3, 1)}
    return out


# ------------------------------------------------------------------ CPU side

def cpu_threads():
    """Threads for the CPU oracle: the host's cores available to this
    process, capped by OMP_NUM_THREADS when the environment sets it (a
    host shared by several GPUs' jobs gives each a share of its cores)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_plan_model(det_g, det_x, rec_x, stage_ms, ctx, ctx_rec, stream, stream_rec, both_sync,
                    report_path):
    """The headline graphs as the reference's plan model runs them: each
    graph lowered to a GraphPlan (qppocr_amd.plan, PlanBuilder's Vulkan
    configuration: rec with the pairs exit, no fused head) and replayed
    alone on its stream, HIP events around the replays (inputs resident)."""
    from qppocr_amd import nets, plan
    rec_g, _ = nets.build_rec(3, REC_BATCH, 320, probs=False)
    out = {"workload": "det 1x3x640x640 and rec 32x3x48x320 (pairs exit) as GraphPlans on the "
                       "n_* kernel set",
           "method": "HIP events over the timed replays of each plan alone (word 0 and the "
                     "graph launch per replay)"}
    plans = {}
    for name, g, x, c, st in (("det", det_g, det_x, ctx, stream),
                              ("rec", rec_g, rec_x, ctx_rec, stream_rec)):
        pl = plan.build_plan(g)
        sess = plan.HipPlanSession(pl, ctx=c)
        sess.run(x, outputs=False)
        sess.run(None, outputs=False)
        both_sync()
        ms = stage_ms(sess, st)
        out[name + "_ms"] = round(ms, 4)
        out[name + "_dispatches"] = len(pl.dispatches)
        out[name + "_launches"] = sess.launches()
        out[name + "_arena_mib"] = round(pl.total_words * 4 / 2 ** 20, 1)
        plans[name] = [[d[0], d[3]] for d in pl.dispatches]
        sess.close()
    out["det_img_per_s"] = round(1e3 / out["det_ms"], 2)
    out["rec_lines_per_s"] = round(REC_BATCH * 1e3 / out["rec_ms"], 1)
    if report_path:
        with open(report_path, "w") as f:
            json.dump(plans, f)
    return out


def cpu_sample(fn, rounds, min_s=0.0):
    """One warm-up round, then timed rounds until at least `rounds` have run
    and together they took `min_s` seconds (the reference CLI bench
    discipline, qppocr-cli/src/main.rs:738-818, with a time floor so the
    sample is some seconds of CPU work).  Returns (median seconds, rounds)."""
    fn()
    ts = []
    while len(ts) < rounds or (sum(ts) < min_s and len(ts) < 1000000):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), len(ts)


# ------------------------------------------------------------------ GPU side

class ColdOpBench:
    """One op as a session node with resident weights, copied over R input /
    output buffer sets (R x set bytes > COLD_BYTES); a graph replay runs the
    copies back to back.  add_node(g, x) appends the op reading tensor x.
    warm=True: the R copies all read the same input instead (back-to-back
    launches on cache-resident data)."""

    def __init__(self, nets, ops, ctx, x, add_node, set_bytes, warm=False):
        import numpy as np
        self.R = max(2, -(-COLD_BYTES // set_bytes))
        g = nets.Graph(x.shape)
        ins = [0] * self.R if warm else [0] + [g.tensor(x.shape) for _ in range(self.R - 1)]
        outs = [add_node(g, t) for t in ins]
        g.outputs = [outs[0]]
        g.flags = nets.NET_SEPARATE_LAUNCHES     # one launch per copy
        self.g = g
        self.sess = nets.HipSession(g, ctx=ctx)
        self.sess.run(x, outputs=False)
        xc = np.ascontiguousarray(x, dtype=np.float32)
        lib = ops._lib.load()
        for t in ([] if warm else ins[1:]):
            ptr, n = self.sess.tensor_ptr(t)
            ops.check(lib.qph_memcpy_h2d(ctx, ctypes.c_void_p(ptr),
                                         xc.ctypes.data_as(ctypes.c_void_p), n * 4))
        self.stream = lib.qph_ctx_stream(ctx)

    def us_per_launch(self, replays, warmup=2):
        import torch
        st = torch.cuda.ExternalStream(self.stream)
        for _ in range(warmup):
            self.sess.run(None, outputs=False)
        self.sess.sync()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(replays):
            self.sess.run(None, outputs=False)
        e1.record(st)
        self.sess.sync()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (replays * self.R)

    def close(self):
        self.sess.close()


def bench_cfg1(nets, ops, configs, ctx, replays, cpu_rounds, O):
    from qppocr_amd._lib import ACT_RELU
    x, w, b = configs.cfg1(0)
    by, fl = configs.cfg1_bytes_flops()

    def add_node(g, t):
        if not g.weights:        # weight ids 0 (w) and 1 (bias), shared by the copies
            g.weight(w)
            g.weight(b)
        return g.conv(t, 0, 1, pad=(1, 1, 1, 1), act=ACT_RELU)
    set_bytes = x.nbytes + 4 * 32 * 160 * 160
    ob = ColdOpBench(nets, ops, ctx, x, add_node, set_bytes, warm=True)
    us = ob.us_per_launch(replays)
    ob.close()
    ob = ColdOpBench(nets, ops, ctx, x, add_node, set_bytes)
    us_cold = ob.us_per_launch(replays)
    ob.close()
    tf = fl / (us * 1e-6) / 1e12
    out = {"workload": "conv3x3 s1 p1 N=1 32->32 160x160 + bias + ReLU (seed 0)",
           "us": round(us, 3), "tflops": round(tf, 2), "bound": "mfma",
           "frac": round(tf / PEAK_FP32_MFMA_TFLOPS, 4), "gflop": round(fl / 1e9, 4),
           "kernel": "conv3x3_lds32_kernel<2>",
           "method": f"HIP events over {replays} graph replays of {ob.R} back-to-back "
                     f"launches on the same input (device time per launch)",
           "us_cache_cold": round(us_cold, 3),
           "cold_method": f"the same over {ob.R} rotating buffer sets "
                          f"({ob.R * set_bytes >> 20} MB, past the 256 MB Infinity Cache)"}
    if O is not None:
        params = O.conv_params(1, 1, 1, 1)
        s, n = cpu_sample(lambda: O.conv2d(x, w, b, params, O.ACT_RELU), cpu_rounds,
                          CPU_CONFIG_MIN_S)
        out["cpu_baseline"] = {"us": round(s * 1e6, 1),
                               "tflops": round(fl / s / 1e12, 4), "rounds": n}
    return out


def stream_floor_us(n_in, n_out, replays):
    """Per-launch time of torch's own device copy streaming the same bytes
    cache-cold (n_in floats read, n_out written: a plain copy when the sizes
    are equal, else a copy of every (n_in / n_out)-th input, which reads
    every cache line of the input), R rotating buffer sets past COLD_BYTES,
    R launches per graph replay: the floor for moving an op's compulsory
    bytes in one launch in this harness."""
    import torch
    set_bytes = 4 * (n_in + n_out)
    R = max(2, -(-COLD_BYTES // set_bytes))
    xs = [torch.rand(n_in, device="cuda") for _ in range(R)]
    ys = [torch.empty(n_out, device="cuda") for _ in range(R)]
    ratio = n_in // n_out

    def body():
        for x, y in zip(xs, ys):
            if ratio == 1:
                y.copy_(x)
            else:
                y.copy_(x.view(n_out, ratio)[:, 0])
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        body()
    st.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        body()
    with torch.cuda.stream(st):
        for _ in range(2):
            gr.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(replays):
            gr.replay()
        e1.record(st)
    st.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * R)
    del gr, xs, ys
    return us


def bench_cfg2(nets, ops, configs, ctx, replays, cpu_rounds, O):
    from qppocr_amd._lib import ACT_HARDSWISH
    res = {}
    for tag, (x, w, b, k, s) in zip("abcd", configs.cfg2(1)):
        c, hw = x.shape[1], x.shape[2]
        by, fl = configs.cfg2_bytes_flops(c, hw, k, s)
        oh = configs.conv_out_hw(hw, k, s, k // 2)

        def add_node(g, t, w=w, b=b, k=k, s=s, c=c):
            if not g.weights:
                g.weight(w)
                g.weight(b)
            return g.conv(t, 0, 1, stride=(s, s), pad=(k // 2,) * 4, group=c, act=ACT_HARDSWISH)
        set_bytes = x.nbytes + 4 * c * oh * oh
        ob = ColdOpBench(nets, ops, ctx, x, add_node, set_bytes)
        us = ob.us_per_launch(replays)
        ob.close()
        gbs = by / (us * 1e-6) / 1e9
        floor = stream_floor_us(x.size, c * oh * oh, replays)
        out = {"workload": f"depthwise {k}x{k} s{s} pad {k // 2} C{c} {hw}x{hw} + hardswish",
               "us": round(us, 3), "gbs": round(gbs, 1), "bound": "hbm",
               "frac": round(gbs / PEAK_HBM_GBS, 4), "mb": round(by / 1e6, 3),
               "kernel": f"depthwise_rows_kernel<{k},{s}>",
               "method": f"cache-cold: HIP events over {replays} graph replays of {ob.R} copies "
                         f"on rotating buffer sets ({ob.R * set_bytes >> 20} MB)",
               "stream_floor_us": round(floor, 3),
               "floor_method": "torch's device copy reading the input bytes and writing the "
                               "output bytes (for the stride-2 cases every 4th input, which "
                               "touches every line of the input), timed the same way: one "
                               "launch's floor for these bytes",
               "frac_of_floor": round(floor / us, 3)}
        if O is not None:
            params = O.conv_params(s, s, k // 2, k // 2, group=c)

            def run_cpu(x=x, w=w, b=b, params=params):
                y = O.conv2d(x, w, b, params)
                return O.binary_flat(y, O.hardsigmoid(y), 2)
            sec, n = cpu_sample(run_cpu, cpu_rounds, CPU_CONFIG_MIN_S)
            out["cpu_baseline"] = {"us": round(sec * 1e6, 1), "gbs": round(by / sec / 1e9, 2),
                                   "rounds": n}
        res["cfg2" + tag] = out
    return res


def aux_specs(torch, lib, ctx):
    """The operators around the nets, each at a page-scale shape (the mixed
    page's det size 1536^2 and a 32-line rec batch): (name, workload, kernel,
    make_set, call, launches per set, algorithmic bytes per set, cpu).
    make_set() allocates one input / output buffer set, call(s) issues its
    launches on ctx's stream, cpu(O, h) runs the oracle's work for the same
    set (host arrays h)."""
    P = ctypes.c_void_p
    I64 = ctypes.c_int64

    def u8(*shape):
        return torch.randint(0, 256, shape, dtype=torch.uint8, device="cuda")

    def f32(*shape):
        return torch.rand(shape, device="cuda")

    def ptr(t):
        return P(t.data_ptr())

    def nb(*ts):
        return sum(t.numel() * t.element_size() for t in ts)
    specs = []
    # page image -> det input size (resize.rs:153-209)
    specs.append(("resize_rgb_u8", "u8 RGB 2048x2048 -> 1536x1536 bilinear",
                  "resize_rgb_u8_kernel", lambda: (u8(2048, 2048, 3), u8(1536, 1536, 3)),
                  lambda s: lib.qph_resize_bilinear_rgb_u8(ctx, ptr(s[0]), 2048, 2048, ptr(s[1]),
                                                           1536, 1536), 1, nb,
                  lambda O, h: O.resize_bilinear_rgb_u8(h[0], 1536, 1536)))
    # det input normalisation (engine.rs:959-982)
    specs.append(("det_normalize_u8", "u8 RGB 1536x1536 -> f32 1x3x1536x1536 ((v/255-0.5)/0.5)",
                  "det_normalize_kernel", lambda: (u8(1536, 1536, 3), f32(1, 3, 1536, 1536)),
                  lambda s: lib.qph_det_normalize_u8(ctx, ptr(s[0]), 1536, 1536, ptr(s[1])), 1,
                  nb, lambda O, h: O.det_normalize(h[0])))

    # rec line packing (crop.rs:153-190): 32 crops of 40x240 into 3x48x320 slots
    def crops():
        return tuple(u8(40, 240, 3) for _ in range(32)) + (f32(32, 3, 48, 320),)

    def pack(s):
        for i in range(32):
            r = lib.qph_pack_crop(ctx, ptr(s[i]), 40, 240, 48, 320, 0,
                                  P(s[32].data_ptr() + i * 3 * 48 * 320 * 4))
            if r != 0:
                return r
        return 0
    def pack_cpu(O, h):
        for i in range(32):
            O.pack_crop(h[i], 48, 320, False)
    specs.append(("pack_crop", "32 u8 RGB crops 40x240 -> f32 32x3x48x320 (resized to 48x288, "
                  "zero tail), one launch per line", "pack_crop_kernel", crops, pack, 32, nb, pack_cpu))
    ptrs = {}

    def pack_batch(s):
        # the descriptor arrays of a set, built once (host memory, read at launch)
        key = s[32].data_ptr()
        if key not in ptrs:
            ptrs[key] = ((ctypes.c_void_p * 32)(*[t.data_ptr() for t in s[:32]]),
                         (I64 * 32)(*([40] * 32)), (I64 * 32)(*([240] * 32)),
                         (ctypes.c_int32 * 32)())
        cp, ch, cw, po = ptrs[key]
        return lib.qph_pack_crops(ctx, 32, cp, ch, cw, po, 48, 320, ptr(s[32]))
    specs.append(("pack_crops", "the same 32 lines in one launch (the batch entry point)",
                  "pack_crops_kernel", crops, pack_batch, 1, nb, pack_cpu))
    # DB threshold + 2x2 dilation (geometry.rs:287-301, resize.rs:219-247)
    specs.append(("db_mask", "f32 probability map 1536x1536 -> u8 mask, thresh 0.3, dilated",
                  "db_mask_kernel", lambda: (f32(1536, 1536), u8(1536, 1536)),
                  lambda s: lib.qph_db_mask(ctx, ptr(s[0]), 1536, 1536, ctypes.c_float(0.3), 1,
                                            ptr(s[1])), 1, nb,
                  lambda O, h: O.db_mask(h[0], 0.3, True)))
    # SE squeeze and excite (pool2d.rs:10-29, elementwise.rs:134-179)
    specs.append(("global_avg_pool", "f32 1x256x96x96 -> 1x256 (f64 mean per plane)",
                  "reduce_mean_wg_kernel<true>", lambda: (f32(1, 256, 96, 96), f32(256)),
                  lambda s: lib.qph_global_avg_pool(ctx, ptr(s[0]), 1, 256, 96 * 96, ptr(s[1])),
                  1, nb, lambda O, h: O.global_avg_pool(h[0])))
    specs.append(("mul_add_scale", "f32 1x256x96x96 * gate[256] + residual",
                  "mul_add_scale_kernel",
                  lambda: (f32(1, 256, 96, 96), f32(256), f32(1, 256, 96, 96),
                           f32(1, 256, 96, 96)),
                  lambda s: lib.qph_mul_add_scale(ctx, ptr(s[0]), ptr(s[1]), ptr(s[2]), 1, 256,
                                                  96 * 96, ptr(s[3])), 1, nb,
                  lambda O, h: O.mul_add_scale(h[0], h[1], h[2])))
    # MaxPool (pool2d.rs:94-236)
    xs_pool = (I64 * 4)(32, 64, 48, 160)
    ys_pool = (I64 * 4)()
    specs.append(("pool2d_max", "f32 32x64x48x160 -> 32x64x24x80, max 2x2 stride 2",
                  "pool2d_kernel<2>", lambda: (f32(32, 64, 48, 160), f32(32, 64, 24, 80)),
                  lambda s: lib.qph_pool2d(ctx, ptr(s[0]), xs_pool, 2, 2, 2, 2, 0, 0, 0, 0, 1,
                                           ptr(s[1]), ys_pool), 1, nb,
                  lambda O, h: O.pool2d(h[0], 2, 2, 2, 2, 0, 0, 0, 0, True)))
    # bilinear Resize (resize.rs:60-142): a det map back to page size
    specs.append(("resize_bilinear", "f32 1x1x384x384 -> 1536x1536 (half-pixel)",
                  "resize_bilinear_kernel", lambda: (f32(384, 384), f32(1536, 1536)),
                  lambda s: lib.qph_resize_bilinear(ctx, ptr(s[0]), 1, 384, 384, 1536, 1536, 0,
                                                    ptr(s[1])), 1, nb,
                  lambda O, h: O.resize_bilinear(h[0], 1536, 1536, False)))
    xs_tr = (I64 * 4)(1, 96, 384, 384)
    perm = (ctypes.c_int32 * 4)(0, 2, 3, 1)
    specs.append(("transpose", "f32 1x96x384x384 -> 1x384x384x96 (NCHW -> NHWC)",
                  "transpose4_tile_kernel", lambda: (f32(1, 96, 384, 384), f32(1, 384, 384, 96)),
                  lambda s: lib.qph_transpose(ctx, ptr(s[0]), xs_tr, perm, ptr(s[1])), 1, nb,
                  lambda O, h: O.transpose4(h[0], (0, 2, 3, 1))))
    return specs


def bench_cls(nets, lib, torch, ctx, replays, cpu_rounds, O):
    """The cls stage's net (the orientation classifier of engine.rs:1294-1380)
    on a full batch of 32 lines of 3x48x192: HIP events around graph replays
    on the session's stream; the CPU oracle beside it."""
    g, x = nets.build_cls(5, 32)
    sess = nets.HipSession(g, ctx=ctx)
    sess.run(x, outputs=False)
    for _ in range(3):
        sess.run(None, outputs=False)
    sess.sync()
    st = torch.cuda.ExternalStream(lib.qph_ctx_stream(ctx))
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(replays):
        sess.run(None, outputs=False)
    e1.record(st)
    e1.synchronize()
    ms = e0.elapsed_time(e1) / replays
    out = {"workload": "cls 32x3x48x192 (seed 5), probabilities", "lines_per_s": round(32e3 / ms, 1),
           "ms": round(ms, 4), "gflop": round(nets.flops(g) / 1e9, 4),
           "launches": len(sess.plan()), "method": f"HIP events over {replays} graph replays"}
    sess.close()
    if O is not None:
        from oracle import nets as onets
        s, n = cpu_sample(lambda: onets.run_graph(g, x), cpu_rounds, CPU_CONFIG_MIN_S)
        out["cpu_baseline"] = {"lines_per_s": round(32 / s, 2), "rounds": n}
    return out


def bench_aux(ops, replays, O=None, cpu_rounds=5):
    """Device time per launch of the operators around the nets (aux_specs),
    cache-cold: R buffer sets (R x set bytes > COLD_BYTES) whose launches are
    captured once into a graph, replayed `replays` times between HIP events.
    With the oracle O: its time on the same set beside each (median of the
    rounds in >= CPU_AUX_MIN_S, per launch)."""
    import torch
    lib = ops._lib.load()
    ctx = ops.new_context(0)
    st = torch.cuda.Stream()
    ops.check(lib.qph_ctx_set_stream(ctx, ctypes.c_void_p(st.cuda_stream)))
    torch.manual_seed(5)
    out = {}
    try:
        for name, workload, kernel, make, call, nl, nbytes, cpu in aux_specs(torch, lib, ctx):
            first = make()
            set_bytes = nbytes(*first)
            R = max(2, -(-COLD_BYTES // set_bytes))
            sets = [first] + [make() for _ in range(R - 1)]
            torch.cuda.synchronize()
            with torch.cuda.stream(st):
                for s in sets:
                    ops.check(call(s))
            st.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=st):
                for s in sets:
                    ops.check(call(s))
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(st):
                graph.replay()
                e0.record(st)
                for _ in range(replays):
                    graph.replay()
                e1.record(st)
            e1.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (replays * R * nl)
            by = set_bytes / nl
            gbs = by / (us * 1e-6) / 1e9
            out[name] = {"workload": workload, "kernel": kernel, "us": round(us, 3),
                         "mb": round(by / 1e6, 4), "gbs": round(gbs, 1), "bound": "hbm",
                         "frac": round(gbs / PEAK_HBM_GBS, 4),
                         "method": f"cache-cold: HIP events over {replays} replays of a graph "
                                   f"of {R * nl} launches on {R} rotating buffer sets "
                                   f"({R * set_bytes >> 20} MB)"}
            if O is not None:
                h = [t.cpu().numpy() for t in first]
                sec, n = cpu_sample(lambda: cpu(O, h), cpu_rounds, CPU_AUX_MIN_S)
                out[name]["cpu_baseline"] = {"us": round(sec * 1e6 / nl, 1),
                                             "gbs": round(by / (sec / nl) / 1e9, 2), "rounds": n}
            del graph, sets, first
            torch.cuda.synchronize()
    finally:
        ops.check(lib.qph_ctx_set_stream(ctx, None))
        ops.close_context(ctx)
    return out


def time_mixed_page(steps, warmup, engine=False, data=None):
    """det 1x3x1536x1536 + 128 rec lines (widths {80..1280}, buckets of 160,
    <= 64 lines per batch, fused rec heads), inputs resident.  det and the rec batches run on
    three streams (det; rec batches alternating over two): page_ms is the
    wall time per page over the steps; det_ms / rec_ms are each stage alone.
    engine: the lines batched as the reference engine batches them for a GPU
    session (spans of 64 px, 64 lines a forward, widths rounded to 64), each
    batch on a 64-row net run with real_n = its line count."""
    import numpy as np
    import torch
    from qppocr_amd import ops, pipeline
    det_g, det_x, rw, lines, widths = data if data else pipeline.mixed_page(4, 1536, 128)
    ctxs = [ops.new_context(0) for _ in range(3)]
    page = pipeline.PageRunner(det_g, det_x, rw, lines, widths, contexts=ctxs, fused_head=True,
                               engine=engine)
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
    creates = page.net_create_ms
    out = {"workload": ("det 1x3x1536x1536 + 128 rec lines 3x48x{80..1280}, engine batching "
                        "(spans of 64 px, <= 64 lines a forward, widths to 64, batch padded to "
                        "64 with real_n), CTC masked past w/8 (seed 4)") if engine else
                       ("det 1x3x1536x1536 + 128 rec lines 3x48x{80..1280}, buckets of 160, "
                        "<= 64 lines/batch, CTC masked past w/8 (seed 4)"),
           "rec_batches": [[bw, len(idx)] for bw, idx in page.plan],
           "rec_net_create_ms": {"n": len(creates),
                                 "mean": round(float(np.mean(creates)), 2),
                                 "max": round(float(np.max(creates)), 2)},
           "det_img_per_s": round(1e3 / det_ms, 2),
           "rec_lines_per_s": round(len(widths) * 1e3 / rec_ms, 1),
           "page_ms": round(page_ms, 4), "ms_per_image": round(page_ms, 4),
           "det_ms": round(det_ms, 4), "rec_ms": round(rec_ms, 4)}
    page.close()
    for c in ctxs:
        ops.close_context(c)
    return out, (det_g, det_x, rw, lines, widths)


def cpu_mixed_page(data, rounds):
    """The mixed page on the CPU oracle: det at 1536^2 and every rec batch."""
    from qppocr_amd import nets, pipeline
    from oracle import nets as onets
    det_g, det_x, rw, lines, widths = data
    batches = [(nets.build_rec_graph(rw, len(idx), bw, pipeline.REC_H, probs=False),
                pipeline.pack_lines(lines, idx, bw)) for bw, idx in pipeline.bucket_plan(widths)]
    det_s, det_n = cpu_sample(lambda: onets.run_graph(det_g, det_x), rounds, CPU_CONFIG_MIN_S)

    def rec():
        for g, x in batches:
            onets.run_graph(g, x)
    rec_s, rec_n = cpu_sample(rec, rounds, CPU_CONFIG_MIN_S)
    return {"det_img_per_s": round(1.0 / det_s, 3),
            "rec_lines_per_s": round(len(widths) / rec_s, 2),
            "ms_per_image": round((det_s + rec_s) * 1e3, 1), "rounds": [det_n, rec_n]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--pages-in-flight", type=int, default=2,
                    help="pages the timed headline keeps in flight, each on its own det and rec "
                         "session (two streams a page; 2 fills the 4 hardware queues)")
    ap.add_argument("--cpu-rounds", type=int, default=5,
                    help="CPU baseline: least timed rounds (median) after one warm-up round; "
                         "more run until the leg's time floor is reached")
    ap.add_argument("--no-configs", action="store_true",
                    help="headline step only (skip the per-config measurements)")
    ap.add_argument("--node-report", default="",
                    help="also write per-node work, eager per-node times and the launch plans "
                         "of the headline graphs (JSON) to this path")
    ap.add_argument("--no-plan", action="store_true",
                    help="skip the plan-model leg (the headline graphs as GraphPlans)")
    ap.add_argument("--plan-only", action="store_true",
                    help="run only the plan-model leg and print its figures (profiling)")
    ap.add_argument("--plan-report", default="",
                    help="write the plan-model graphs' dispatch lists (JSON) to this path")
    ap.add_argument("--aux-only", action="store_true",
                    help="run only the leg of the operators around the nets (profiling)")
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
    from qppocr_amd import configs, nets, ops

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if args.aux_only:
        print(json.dumps({"aux": bench_aux(ops, max(3, min(args.steps, 50) // 5))}))
        return
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
    rec_g, rec_x = nets.build_rec(3, REC_BATCH, 320, fused_head=True)
    if args.plan_only:
        # the plan-model leg alone (for kernel traces of the plan path)
        def sync_all():
            ops.check(lib.qph_sync(ctx))
            ops.check(lib.qph_sync(ctx_rec))
            torch.cuda.synchronize()

        def stage(sess, st):
            for _ in range(args.warmup):
                sess.run(None, outputs=False)
            sync_all()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(st)
            for _ in range(args.steps):
                sess.run(None, outputs=False)
            e1.record(st)
            sync_all()
            return e0.elapsed_time(e1) / args.steps
        leg = time_plan_model(det_g, det_x, rec_x, stage, ctx, ctx_rec, stream, stream_rec,
                              sync_all, args.plan_report)
        print(json.dumps({"plan_model": leg, "steps": args.steps, "warmup": args.warmup}))
        return
    # the other pages in flight: a det and a rec session each, on contexts
    # (streams) of their own.  Every context is created before any session:
    # the HIP runtime hands hardware queues to streams in turn, and creating
    # a session takes queues from the same rotation, so a context created
    # after sessions can share a queue with an earlier stream and run behind it
    P = max(1, args.pages_in_flight)
    extra_ctx = [ops.new_context(0) for _ in range(2 * (P - 1))]
    det = nets.HipSession(det_g, ctx=ctx)
    rec = nets.HipSession(rec_g, ctx=ctx_rec)
    pages = [(det, rec)]
    for j in range(P - 1):
        pages.append((nets.HipSession(det_g, ctx=extra_ctx[2 * j]),
                      nets.HipSession(rec_g, ctx=extra_ctx[2 * j + 1])))
    # inputs resident in HBM: copied once, then every step reuses them
    for d, r in pages:
        d.run(det_x, outputs=False)
        r.run(rec_x, outputs=False)
    for d, r in pages:
        d.sync()
        r.sync()

    def both_sync():
        for d, r in pages:
            d.sync()
            r.sync()
        torch.cuda.synchronize()

    for _ in range(args.warmup):
        for d, r in pages:
            d.run(None, outputs=False)
            r.run(None, outputs=False)
    both_sync()

    K = args.steps

    def stage_ms(sess, st):
        """Each session alone on its own stream: HIP events around K replays."""
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

    # the timed region: K steps (pages), det and rec of each on their
    # streams, page i on session pair i % P: P pages in flight
    both_sync()
    t0 = time.perf_counter()
    for i in range(K):
        d, r = pages[i % P]
        d.run(None, outputs=False)
        r.run(None, outputs=False)
    both_sync()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / K
    # the same K steps with one page in flight (one det and one rec stream)
    both_sync()
    t0 = time.perf_counter()
    for i in range(K):
        det.run(None, outputs=False)
        rec.run(None, outputs=False)
    both_sync()
    t1 = time.perf_counter()
    ms_step_one = (t1 - t0) * 1e3 / K
    for d, r in pages[1:]:
        d.close()
        r.close()
    for c in extra_ctx:
        ops.close_context(c)
    pages = pages[:1]

    # the same step with host buffers at the boundary, through the sessions'
    # pinned staging buffers (deferred runs): det input up and det map down,
    # rec input up and rec pairs down
    det.staging(-1)[:] = det_x
    det.staging(0)
    rec.staging(-1)[:] = rec_x
    rec.staging(0)
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    for _ in range(K):
        det.run_async()
        rec.run_async()
        det.complete()
        rec.complete()
    h1 = time.perf_counter()
    host_ms_step = (h1 - h0) * 1e3 / K

    # the rec graph with the separate head softmax (bit-exact pairs), and
    # that graph exporting the probability tensor as well
    rec_p_g, _ = nets.build_rec(3, REC_BATCH, 320, probs=True)
    rec_p = nets.HipSession(rec_p_g, ctx=ctx_rec)
    rec_p.run(rec_x, outputs=False)
    rec_p.sync()
    rec_p_ms = stage_ms(rec_p, stream_rec)
    rec_p.close()
    rec_e_g, _ = nets.build_rec(3, REC_BATCH, 320, probs=False)
    rec_e = nets.HipSession(rec_e_g, ctx=ctx_rec)
    rec_e.run(rec_x, outputs=False)
    rec_e.sync()
    rec_e_ms = stage_ms(rec_e, stream_rec)
    rec_e.set_profiling(True)
    for _ in range(K):
        rec_e.run(None, outputs=False)
    rec_e.sync()
    e_node_ms = rec_e.node_times()
    rec_e.set_profiling(False)
    rec_e.close()
    e_head = len(rec_e_g.nodes) - 2
    unfused = {"kernel": "rec head GEMM 1280x18709x256 (gemm_wave_kernel<1>)",
               "avg_launch_ms": round(e_node_ms[e_head], 5),
               "softmax_argmax_ms": round(e_node_ms[e_head + 1], 5)}

    # dominant kernel: rec head GEMM, events around each node (eager launches)
    rec.set_profiling(True)
    for _ in range(K):
        rec.run(None, outputs=False)
    rec.sync()
    node_ms = rec.node_times()
    rec.set_profiling(False)
    head = len(rec_g.nodes) - 2        # linear 256 -> 18709 + softmax / argmax
    head_ms = node_ms[head]
    d = rec_g.nodes[head]
    rows = rec_g.numel(d["inp"]) // d["ws"][0]
    head_flops = 2 * rows * d["ws"][0] * d["ws"][1]
    achieved = head_flops / (head_ms * 1e-3) / 1e12
    det.set_profiling(True)
    for _ in range(K):
        det.run(None, outputs=False)
    det.sync()
    det_node_ms = det.node_times()
    det.set_profiling(False)
    plan_leg = None
    if not args.no_plan:
        plan_leg = time_plan_model(det_g, det_x, rec_x, stage_ms, ctx, ctx_rec, stream, stream_rec,
                                   both_sync, args.plan_report)
    if args.node_report:
        # per-node work and eager event times, and each graph's launch plan
        # (for matching a kernel trace of the replays: qppocr_amd.trace_report)
        with open(args.node_report, "w") as f:
            json.dump({"det": {"nodes": node_rows(nets, "det", det_g, det_node_ms),
                               "plan": det.plan()},
                       "rec": {"nodes": node_rows(nets, "rec", rec_g, node_ms),
                               "plan": rec.plan()}}, f, indent=0)

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
        "config": {"workload": "det 1x3x640x640 + rec 32x3x48x320 per step, "
                               "rec ending in the CTC (value, index) pairs",
                   "pages_in_flight": P,
                   "det_gflop": round(det_flops / 1e9, 3), "rec_gflop": round(rec_flops / 1e9, 3)},
        "det_img_per_s": round(1e3 / det_ms, 2),
        "rec_lines_per_s": round(REC_BATCH * 1e3 / rec_ms, 1),
        "rec_lines_per_s_bitexact_pairs": round(REC_BATCH * 1e3 / rec_e_ms, 1),
        "rec_lines_per_s_with_probs": round(REC_BATCH * 1e3 / rec_p_ms, 1),
        "det_ms": round(det_ms, 4),
        "rec_ms": round(rec_ms, 4),
        "serial_ms_per_step": round(det_ms + rec_ms, 4),
        "one_page_in_flight": {"value": round(1e3 / ms_step_one, 3),
                               "ms_per_step": round(ms_step_one, 4)},
        "pcie_inclusive_img_per_s": round(1e3 / host_ms_step, 3),
        "roofline": {"bound": "mfma",
                     "kernel": "fused rec head: GEMM 1280x18709x256 + softmax/argmax epilogue "
                               "(gemm_wave_kernel<2> + head_pairs_kernel)",
                     "achieved": round(achieved, 2), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
                     "traffic": head_traffic_bytes(), "avg_launch_ms": round(head_ms, 5)},
        "head_gemm_unfused": dict(unfused, **{
            "frac": round(head_flops / (unfused["avg_launch_ms"] * 1e-3) / 1e12
                          / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": head_traffic_bytes("rec_head_gemm_traffic.md")}),
    }
    if plan_leg is not None:
        result["plan_model"] = plan_leg

    O = None
    threads = None
    if not args.no_cpu:
        from oracle import nets as onets
        from oracle import oracle as O
        O.lib()
        threads = cpu_threads()
        O.set_threads(threads)

    cfgs = {}
    if not args.no_configs:
        reps = max(3, min(K, 50) // 5)
        cfgs["cfg1"] = bench_cfg1(nets, ops, configs, ctx, reps, args.cpu_rounds, O)
        cfgs.update(bench_cfg2(nets, ops, configs, ctx, reps, args.cpu_rounds, O))
    cfgs["cfg3"] = {"workload": "det 1x3x640x640 (seed 2)", "img_per_s": result["det_img_per_s"],
                    "ms": result["det_ms"], "gflop": round(det_flops / 1e9, 3),
                    "classes": class_fractions(nets, det_g, det_node_ms)}
    cfgs["cfg4"] = {"workload": "rec 32x3x48x320 (seed 3), pairs exit (fused head)",
                    "lines_per_s": result["rec_lines_per_s"], "ms": result["rec_ms"],
                    "gflop": round(rec_flops / 1e9, 3),
                    "classes": class_fractions(nets, rec_g, node_ms)}
    mixed_data = None
    if not args.no_configs:
        cfgs["cfg5"], mixed_data = time_mixed_page(max(3, min(K, 50) // 5), 2)
        cfgs["cfg5"]["engine_batching"], _ = time_mixed_page(max(3, min(K, 50) // 5), 2, engine=True,
                                                             data=mixed_data)
        cfgs["cls"] = bench_cls(nets, lib, torch, ctx, max(3, min(K, 50) // 2), args.cpu_rounds, O)

    if O is not None:
        det_s, det_n = cpu_sample(lambda: onets.run_graph(det_g, det_x), args.cpu_rounds,
                                  CPU_HEADLINE_MIN_S)
        rec_s, rec_n = cpu_sample(lambda: onets.run_graph(rec_g, rec_x), args.cpu_rounds,
                                  CPU_HEADLINE_MIN_S)
        cfgs["cfg3"]["cpu_baseline"] = {"img_per_s": round(1.0 / det_s, 3), "rounds": det_n}
        cfgs["cfg4"]["cpu_baseline"] = {"lines_per_s": round(REC_BATCH / rec_s, 2),
                                        "rounds": rec_n}
        if mixed_data is not None:
            cfgs["cfg5"]["cpu_baseline"] = cpu_mixed_page(mixed_data, args.cpu_rounds)
        result["cpu_baseline"] = {
            "value": round(1.0 / (det_s + rec_s), 4),
            "unit": result["unit"],
            "cores": threads,
            "kind": "port",
            "sample": f"det 1x3x640x640 and rec 32x3x48x320 (pairs exit) on the CPU oracle, each "
                      f"1 warm-up + median of the rounds in >= {CPU_HEADLINE_MIN_S:.0f} s "
                      f"({det_n} det, {rec_n} rec rounds; {det_s:.4f} + {rec_s:.4f} "
                      f"s per step), OpenMP {threads} threads of {os.cpu_count()} logical CPUs "
                      f"({cpu_model()}), -O3 -mavx2 -mfma, FTZ/DAZ",
        }
    result["configs"] = cfgs
    if not args.no_configs:
        result["aux"] = bench_aux(ops, max(3, min(K, 50) // 5), O, args.cpu_rounds)
    print(json.dumps(result))
    det.close()
    rec.close()
    ops.close_context(ctx_rec)


if __name__ == "__main__":
    main()
