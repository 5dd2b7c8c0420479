"""The kernel-trace roofline report (qppocr_amd.trace_report) on a synthetic
trace: replay selection and the work booked per launch."""
import csv
import json

from qppocr_amd import trace_report as tr

FIELDS = ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Stream_Id",
          "Start_Timestamp", "End_Timestamp"]


class Trace:
    """Kernels laid out back to back per stream, in nanoseconds."""

    def __init__(self):
        self.rows = []
        self.t = {}

    def run(self, stream, names, dur=1000, gap=100, at=None):
        t = self.t.get(stream, 0) if at is None else at
        for n in names:
            self.rows.append({"Kernel_Name": f"void qph::{n}(float const*)", "Grid_Size_X": "64",
                              "Grid_Size_Y": "1", "Grid_Size_Z": "1", "Stream_Id": str(stream),
                              "Start_Timestamp": str(t), "End_Timestamp": str(t + dur)})
            t += dur + gap
        self.t[stream] = t

    def idle(self, stream, ns=100000):
        self.t[stream] = self.t.get(stream, 0) + ns


GRAPH_A = ["k_stem", "k_mid", "k_head<2>", "k_pairs"]     # fused head: 3 launches
GRAPH_B = ["k_stem", "k_mid", "k_head<1>", "k_softmax"]   # same kernel count


def nodes_json():
    nodes = [
        {"op": "conv", "gflop": 1.0, "mb": 10.0, "t_in": 0, "t_out": 1, "in_mb": 2.0, "out_mb": 3.0},
        {"op": "conv", "gflop": 2.0, "mb": 20.0, "t_in": 1, "t_out": 2, "in_mb": 3.0, "out_mb": 4.0},
        {"op": "linear", "gflop": 4.0, "mb": 50.0, "t_in": 2, "t_out": 3, "in_mb": 4.0,
         "out_mb": 30.0},
        {"op": "softmax_argmax", "gflop": 0.0, "mb": 31.0, "t_in": 3, "t_out": 4,
         "in_mb": 30.0, "out_mb": 1.0},
    ]
    return {"nodes": nodes, "plan": [(0, 1, 1), (1, 1, 1), (2, 2, 2)]}


GRAPH_C = ["c0", "c1", "c2", "c3", "c4", "c5"]   # 6 kernels: cut by 4 it repeats every 12


def test_takes_the_earliest_graph_and_drops_internal_tensors(tmp_path):
    t = Trace()
    for _ in range(6):                       # an earlier graph of another kernel count
        t.run(0, GRAPH_C, dur=2000)
    t.idle(0)
    t.run(0, GRAPH_A + ["k_extra"])          # a stretch that is not whole replays
    t.idle(0)
    for _ in range(4):                       # headline graph, replays back to back
        t.run(0, GRAPH_A, dur=1000)
    t.idle(0)
    t.run(0, GRAPH_A, dur=1000)              # overlapped by stream 1: not alone
    t.run(1, ["k_other"], dur=5000, at=int(t.rows[-4]["Start_Timestamp"]))
    t.idle(0)
    for _ in range(6):                       # a later graph of equal kernel count, more replays
        t.run(0, GRAPH_B, dur=3000)
    t.idle(0)
    t.run(0, GRAPH_A, dur=1000, gap=50000)   # eager (gaps between kernels): not a replay
    trace = tmp_path / "run_kernel_trace.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        w.writerows(t.rows)
    rows = list(csv.DictReader(open(trace)))
    reps = tr.alone_replays(rows, 4)
    assert len(reps) == 4
    assert all(tr._name(r[2]) == "k_head<2>" for r in reps)

    lines = tr.summarize("rec", nodes_json(), rows)
    head = [ln for ln in lines if "k_head<2> + k_pairs" in ln][0].split("|")
    # 2 kernels of 1000 ns; 4 GFLOP; 50 + 31 MB less the logits (30 written + 30 read)
    assert float(head[5]) == 2.0
    assert abs(float(head[6]) - 4.0) < 1e-9
    assert abs(float(head[7]) - 21.0) < 1e-9
    assert "3 launches (4 kernels), 4 replays" in lines[0]


def test_internal_mb_needs_a_reader_inside_the_launch():
    n = nodes_json()["nodes"]
    assert tr.internal_mb(n[:1]) == 0.0
    assert tr.internal_mb(n[0:2]) == 3.0 + 3.0
    assert tr.internal_mb(n[0:3]) == (3.0 + 3.0) + (4.0 + 4.0)
    old = [{k: v for k, v in d.items() if not k.startswith(("t_", "in_", "out_"))} for d in n]
    assert tr.internal_mb(old) == 0.0       # node reports without tensor ids


def test_main_writes_both_graphs(tmp_path, capsys):
    t = Trace()
    for _ in range(4):
        t.run(0, ["d0", "d1"])
    t.idle(0)
    for _ in range(4):
        t.run(0, GRAPH_A)
    t.run(0, GRAPH_A[:2])                    # the tracer's idle gap inside a replay:
    t.idle(0, 40000)                         # still one replay, not a back-to-back one
    t.run(0, GRAPH_A[2:])
    t.run(0, ["d0"])
    trace = tmp_path / "t.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        w.writerows(t.rows)
    det = {"nodes": [{"op": "conv", "gflop": 1.0, "mb": 1.0}] * 2, "plan": [(0, 1, 1), (1, 1, 1)]}
    rep = tmp_path / "nodes.json"
    rep.write_text(json.dumps({"det": det, "rec": nodes_json()}))
    tr.main(["trace_report", str(trace), str(rep)])
    out = capsys.readouterr().out
    assert "### det: 2 launches (2 kernels), 4 replays" in out
    assert "### rec: 3 launches (4 kernels), 4 replays" in out
