"""The profiler stage ranges (ress_amd.trace): off by default, balanced pushes and pops, one
range per stage of a layer's sparse attention in launch order, and ROCm's roctx library loads."""

import pytest
import torch

from ress_amd import budget, synth, trace
from ress_amd.kernels import LayerGrid


class RecordingRoctx:
    """Stands in for the roctx library and records the calls."""

    def __init__(self):
        self.calls = []

    def roctxRangePushA(self, name):
        self.calls.append(("push", name.decode()))
        return 0

    def roctxRangePop(self):
        self.calls.append(("pop", None))
        return 0


@pytest.fixture
def recorder():
    rec = RecordingRoctx()
    was = trace.enabled()
    trace.enable(True, lib=rec)
    yield rec
    trace.enable(was)


def test_ranges_are_off_by_default_and_cost_no_calls():
    rec = RecordingRoctx()
    trace.enable(True, lib=rec)
    trace.enable(False)
    with trace.stage("ress.x"):
        pass
    assert rec.calls == []


def test_ranges_nest_and_pop_on_error(recorder):
    with trace.stage("outer"):
        with pytest.raises(ValueError):
            with trace.stage("inner"):
                raise ValueError("stage failed")
    assert recorder.calls == [("push", "outer"), ("push", "inner"), ("pop", None), ("pop", None)]


def test_a_range_opened_while_off_is_not_popped_after_enable(recorder):
    trace.enable(False)
    s = trace.stage("late")
    with s:
        trace.enable(True, lib=recorder)
    assert recorder.calls == []


def test_the_roctx_library_loads_and_ranges_run_without_a_profiler():
    lib = trace._load()
    assert lib.roctxRangePushA(b"ress.test") >= 0
    assert lib.roctxRangePop() >= 0


@pytest.mark.gpu
def test_layer_stages_are_ranged_in_launch_order(recorder, dev):
    from ress_amd.attention import sparse_global_attention

    q, k, v, meta = synth.make_layer_qkv(4)
    g = LayerGrid(1, 16, 4, meta["P"], meta["S"])
    bud = budget.UniformBudget()
    res = sparse_global_attention(q.to(dev), k.to(dev), v.to(dev), g,
                                  budget_fn=lambda a: bud.num_to_select(0, a, 0.5, 0.9, 1.0))
    torch.cuda.synchronize()
    assert torch.isfinite(res.out).all()
    pushes = [n for op, n in recorder.calls if op == "push"]
    assert pushes == ["ress.prepare_blocks", "ress.pooled_scores", "ress.budget", "ress.select",
                      "ress.sparse_attention"]
    assert sum(op == "pop" for op, _ in recorder.calls) == len(pushes)


def _csv(path, header, rows):
    path.write_text("\n".join([",".join(header)] + [",".join(f'"{v}"' for v in r) for r in rows]) + "\n")


def test_stage_times_ties_kernels_to_the_innermost_range_open_at_launch(tmp_path):
    from ress_amd import stage_times

    _csv(tmp_path / "r_marker_api_trace.csv", ["Function", "Thread_Id", "Start_Timestamp", "End_Timestamp"],
         [["ress.select", 7, 100, 200], ["ress.inner", 7, 150, 180], ["ress.other_thread", 8, 100, 200]])
    _csv(tmp_path / "r_hip_api_trace.csv", ["Correlation_Id", "Thread_Id", "Start_Timestamp"],
         [[1, 7, 120], [2, 7, 160], [3, 7, 250], [4, 8, 130]])
    _csv(tmp_path / "r_kernel_trace.csv", ["Correlation_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"],
         [[1, "void (anonymous namespace)::k_rs_pw<4>(Args)", 1000, 1010],
          [2, "k_select(int)", 1020, 1050], [3, "k_late()", 1060, 1061], [4, "void k_x<1>(int)", 1070, 1072],
          [9, "k_unknown()", 1080, 1084]])
    t = stage_times.stage_times(str(tmp_path), "r")
    assert t["ress.select"][:3] == (1, 1, 10) and dict(t["ress.select"][3]) == {"k_rs_pw": 10}
    assert t["ress.inner"][:3] == (1, 1, 30)
    assert t["ress.other_thread"][:3] == (1, 1, 2)
    assert t[stage_times.OUTSIDE][:3] == (0, 2, 5)  # launched after every range, or no launch record
    assert "ress.inner" in stage_times.report(t)
