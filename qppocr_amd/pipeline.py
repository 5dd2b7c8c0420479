"""Page-level det + rec over the HIP sessions (the mixed-shape workload).

One page: a det forward on the page image, then its text lines recognised in
width buckets.  As the reference engine does (qppocr-core/src/pipeline/
engine.rs:1211-1290 batching, 1450-1493 rec run and decode), lines of one
bucket width run together as one batch, zero-padded on the right to the
bucket width; every (batch, bucket width) shape has its own session (its own
HIP graph), created once and replayed.  The rec sessions export (val, idx)
pairs (DeviceSession::rec_argmax_pairs, device.rs:160-165) and the host
collapses them with ctc_decode_pairs (rec.rs:82-115), reading only the
steps t < w_i / 8 of a line of width w_i (the padding is masked out).
"""
import ctypes

import numpy as np

from . import _lib
from .nets import HipSession, build_det, build_rec_graph, rec_weights, WeightRng

REC_H = 48
REC_STRIDE = 8          # rec time steps per input column: T = w / 8
BUCKET = 160
MAX_BATCH = 64


CLS_THRESH = 0.9       # PipelineConfig cls_thresh (config.rs:158)
CLS_PER_DEVICE = 32    # lines per cls forward on a device session (engine.rs:1313-1319)


def cls_batches(n_lines, per=CLS_PER_DEVICE):
    """The cls stage's batches (engine.rs:1321-1324): consecutive runs of at
    most `per` lines, not padded (a shorter last batch runs at its own size;
    on a HipSession of `per` items that is real_n = its size)."""
    return [(b, min(b + per, n_lines)) for b in range(0, n_lines, per)]


def cls_decisions(probs, thresh=CLS_THRESH):
    """Per line (engine.rs:1375-1380): flip the crop by 180 degrees when
    p1 > p0 and p1 >= thresh; the line's confidence is max(p0, p1).
    probs: [n, 2] float32.  Returns (flip bool [n], confidence float32 [n])."""
    p = np.asarray(probs, dtype=np.float32).reshape(-1, 2)
    p0, p1 = p[:, 0], p[:, 1]
    return (p1 > p0) & (p1 >= np.float32(thresh)), np.maximum(p0, p1)


def ctc_decode_pairs(pairs, t_len):
    """Greedy CTC collapse of (val, idx-bits) pairs over the first t_len
    steps (qppocr-core/src/pipeline/rec.rs:82-115): a step emits its index
    when it is not blank (0) and differs from the previous step's index;
    the confidence is the f64 mean of the emitted values (0 if none)."""
    pairs = np.ascontiguousarray(pairs, dtype=np.float32).reshape(-1, 2)
    idx = pairs[:, 1].view(np.uint32)
    ids = []
    conf_sum = 0.0
    prev = -1
    for t in range(int(t_len)):
        b = int(idx[t])
        if b != 0 and b != prev:
            ids.append(b)
            conf_sum += float(pairs[t, 0])
        prev = b
    conf = np.float32(conf_sum / len(ids)) if ids else np.float32(0.0)
    return ids, float(conf)


def bucket_plan(widths, bucket=BUCKET, max_batch=MAX_BATCH):
    """[(bucket_width, [line indices])]: bucket width = ceil(w / bucket) *
    bucket; the lines of one bucket, in input order, cut into batches of at
    most max_batch."""
    bw = ((np.asarray(widths) + bucket - 1) // bucket) * bucket
    plan = []
    for w in sorted(set(int(v) for v in bw)):
        idx = [i for i in range(len(widths)) if bw[i] == w]
        for s in range(0, len(idx), max_batch):
            plan.append((w, idx[s:s + max_batch]))
    return plan


# The reference GPU sessions' batching hooks (DeviceSession,
# qppocr-core/src/device.rs:139-157; the Vulkan session's values,
# qppocr-gpu/src/vulkan/session.rs:2010-2033): widths rounded up to a
# multiple of 64 (128 and 256 gave misreads there), up to 64 real lines
# merged per forward, and the batch dimension padded to 64 inside the session
# with the real count written before the run.
ENGINE_BUCKET_GRAIN = 64
ENGINE_REC_CHUNK = 64
ENGINE_BATCH_GRAIN = 64
REC_MIN_WIDTH = 16      # PipelineConfig::rec_min_width (qppocr-core/src/pipeline/config.rs:150)


def engine_batches(widths, grain=ENGINE_BUCKET_GRAIN, chunk=ENGINE_REC_CHUNK, img_h=REC_H,
                   min_width=REC_MIN_WIDTH):
    """[(img_w, [line indices])] as the reference engine groups rec lines
    for a session that does not prefer host parallelism
    (qppocr-core/src/pipeline/engine.rs:1211-1290, 1413-1422): lines sorted
    by width / height ratio (stable), a group grows while it has fewer than
    `chunk` lines and its widest line is at most `grain` px wider than its
    first; the batch width is the widest line's (at least min_width),
    rounded up to a multiple of `grain`.  Widths are recovered from the
    ratio in f32 as the engine does ((h * r) as i32)."""
    h = np.float32(img_h)
    ratio = np.asarray(widths, dtype=np.float32) / h
    raw = [int(np.float32(h * r)) for r in ratio]
    order = sorted(range(len(raw)), key=lambda i: float(ratio[i]))
    out = []
    beg = 0
    while beg < len(order):
        end = beg + 1
        w0 = raw[order[beg]]
        while end < len(order) and end - beg < chunk and raw[order[end]] - w0 <= grain:
            end += 1
        ids = order[beg:end]
        max_r = max([np.float32(min_width) / h] + [ratio[i] for i in ids])
        img_w = int(np.float32(h * max_r))
        if grain > 1:
            img_w = (img_w + grain - 1) // grain * grain
        out.append((img_w, ids))
        beg = end
    return out


class HipRecSession:
    """The rec DeviceSession as the reference engine drives it
    (qppocr-core/src/device.rs:125-176): prefers_host_parallelism() false,
    bucket_grain() 64, batch_grain() 64, rec_chunk() 64, rec_argmax_pairs()
    true.  run(x) takes a [bsz, 3, 48, W] batch of real lines; the session
    pads the batch to the grain by running the net of shape
    (ceil(bsz / 64) * 64, W) -- created on first use and kept -- with
    real_n = bsz, so the padded items cost nothing.  net_create_ms records
    the wall time of each net creation (the reference prices its plan
    rebuild at ~10 ms, device.rs:139-141)."""

    def __init__(self, weights, device=0, ctx=None, fused_head=True,
                 batch_grain=ENGINE_BATCH_GRAIN):
        self.weights = weights
        self.device = device
        self.ctx = ctx
        self.fused_head = fused_head
        self.grain = int(batch_grain)
        self.nets = {}
        self.net_create_ms = []

    def prefers_host_parallelism(self):
        return False

    def bucket_grain(self):
        return ENGINE_BUCKET_GRAIN

    def batch_grain(self):
        return self.grain

    def rec_chunk(self):
        return ENGINE_REC_CHUNK

    def rec_argmax_pairs(self):
        return True

    def net_for(self, bsz, img_w, key=0):
        """The net serving bsz real lines of width img_w (key separates two
        batches of one shape that stay resident side by side)."""
        import time
        nb = (int(bsz) + self.grain - 1) // self.grain * self.grain
        k = (nb, int(img_w), key)
        if k not in self.nets:
            t0 = time.perf_counter()
            g = build_rec_graph(self.weights, nb, int(img_w), REC_H, probs=False,
                                fused_head=self.fused_head)
            self.nets[k] = HipSession(g, self.device, ctx=self.ctx)
            self.net_create_ms.append((time.perf_counter() - t0) * 1e3)
        return self.nets[k]

    def run(self, x):
        """[bsz, 3, 48, W] -> [bsz, W / 8, 2] (val, idx-bits) pairs."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        return self.net_for(x.shape[0], x.shape[3]).run(x)[-1]

    def close(self):
        for s in self.nets.values():
            s.close()
        self.nets = {}


def pack_lines(lines, idx, bucket_width):
    """[B, 3, 48, bucket_width] batch of the given lines, zero-padded right."""
    out = np.zeros((len(idx), 3, REC_H, bucket_width), dtype=np.float32)
    for b, i in enumerate(idx):
        out[b, :, :, :lines[i].shape[-1]] = lines[i]
    return out


class PageRunner:
    """det on one page size plus rec sessions for a fixed set of line
    widths; inputs are uploaded once (resident in HBM), run() replays the
    det graph and every rec batch graph.  contexts (optional): the det runs
    on contexts[0] and the rec batches round-robin on the others (each
    context is one stream, so they run concurrently); by default everything
    runs on the device's shared context.  fused_head: the rec sessions run
    the head linear with the softmax / argmax in its epilogue (pairs within
    the 1e-4 tolerance, not bit-exact)."""

    def __init__(self, det_graph, det_input, rec_w, lines, widths, device=0, contexts=None,
                 fused_head=False, engine=False):
        """engine: batch the lines as the reference engine does for a GPU
        session (engine_batches: grain-64 spans, 64 lines a forward) and run
        each batch on a 64-row net with real_n = its line count
        (HipRecSession); otherwise the fixed 160 px buckets of the mixed-page
        workload, each batch on a net of exactly its size."""
        ctxs = list(contexts) if contexts else [None]
        rec_ctxs = ctxs[1:] or ctxs[:1]
        self.det = HipSession(det_graph, device, ctx=ctxs[0])
        self.det_input = det_input
        self.widths = np.asarray(widths, dtype=np.int64)
        self.engine = engine
        self.plan = engine_batches(self.widths) if engine else bucket_plan(self.widths)
        self.rec = []
        self.rec_sessions = []
        self.net_create_ms = []
        seen = {}
        for k, (bw, idx) in enumerate(self.plan):
            ctx = rec_ctxs[k % len(rec_ctxs)]
            x = pack_lines(lines, idx, bw)
            if engine:
                rs = HipRecSession(rec_w, device, ctx=ctx, fused_head=fused_head)
                self.rec_sessions.append(rs)
                key = seen.get(bw, 0)
                seen[bw] = key + 1
                sess = rs.net_for(len(idx), bw, key)
                self.net_create_ms += rs.net_create_ms
                g = sess.graph
            else:
                import time
                t0 = time.perf_counter()
                g = build_rec_graph(rec_w, len(idx), bw, REC_H, probs=False, fused_head=fused_head)
                sess = HipSession(g, device, ctx=ctx)
                self.net_create_ms.append((time.perf_counter() - t0) * 1e3)
            self.rec.append((bw, idx, g, sess, x))
        self.lib = _lib.load()

    def upload(self):
        """Inputs to HBM (one copy per session; real lines only) and one run
        to build the graphs."""
        self.det.run(self.det_input, outputs=False)
        for _, _, _, sess, x in self.rec:
            sess.run(x, outputs=False)
        self.sync()

    def run(self):
        """One page: det + every rec batch, inputs already resident."""
        self.det.run(None, outputs=False)
        for _, _, _, sess, _ in self.rec:
            sess.run(None, outputs=False)

    def run_det(self):
        self.det.run(None, outputs=False)

    def run_rec(self):
        for _, _, _, sess, _ in self.rec:
            sess.run(None, outputs=False)

    def sync(self):
        self.det.sync()
        for _, _, _, sess, _ in self.rec:
            sess.sync()

    def det_map(self):
        g = self.det.graph
        ptr, n = self.det.tensor_ptr(g.outputs[0])
        return self._d2h(ptr, n).reshape(g.lshapes[g.outputs[0]])

    def rec_pairs(self):
        """Per line: its [T_bucket, 2] pairs (unmasked)."""
        out = [None] * len(self.widths)
        for bw, idx, g, sess, _ in self.rec:
            ptr, n = sess.tensor_ptr(g.outputs[-1])
            pairs = self._d2h(ptr, n).reshape(g.lshapes[0][0], bw // REC_STRIDE, 2)
            for b, i in enumerate(idx):
                out[i] = pairs[b]
        return out

    def decode(self):
        """Per line: (ids, confidence) over its unpadded steps."""
        return [ctc_decode_pairs(p, int(w) // REC_STRIDE)
                for p, w in zip(self.rec_pairs(), self.widths)]

    def _d2h(self, ptr, n):
        self.sync()
        host = np.empty(n, dtype=np.float32)
        _lib.check(self.lib.qph_memcpy_d2h(self.det.ctx, host.ctypes.data_as(ctypes.c_void_p),
                                           ctypes.c_void_p(ptr), n * 4))
        return host

    def close(self):
        self.det.close()
        for _, _, _, sess, _ in self.rec:
            sess.close()
        for rs in self.rec_sessions:
            rs.close()


def mixed_page(seed=4, det_hw=1536, n_lines=128):
    """The mixed-shape workload: a det_hw^2 page (det architecture and
    input normalisation of the 640^2 workload; its input and weights from
    build_det(seed)) and n_lines rec lines of height 48 with widths uniform
    on {80, 88, ..., 1280} and U[-1, 1) pixels.  One PCG64(seed) stream
    draws the widths, then the line pixels in line order, then the rec
    weights."""
    r = WeightRng(seed)
    widths = r.rng.choice(np.arange(80, 1281, 8), size=n_lines).astype(np.int64)
    det_g, det_x = build_det(seed, det_hw, det_hw)
    lines = [r.uniform((3, REC_H, int(w)), -1.0, 1.0) for w in widths]
    rw = rec_weights(r)
    return det_g, det_x, rw, lines, widths
