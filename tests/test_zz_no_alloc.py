"""``yapd_attn_paged_block_noalloc`` (split-KV partials in a static device
array) against ``yapd_attn_paged_block`` (caller-provided workspace), both
called through the C ABI: bit-identical outputs on two calls in a row, the
second smaller, plus an unsplit call and the size limit."""

import os
import subprocess
import sys

import pytest
import torch

from test_gpu_attention import build_case, reference
from yapd_amd import kernels
from yapd_amd.paged import AttnPlan

pytestmark = pytest.mark.gpu


def noalloc_fn():
    """The C entry point itself (its ctypes prototype mirrors include/yapd_t3.h)."""
    return kernels.load_library().yapd_attn_paged_block_noalloc


def run_pair(dev, rows, bl, lengths, seed, target, min_split):
    q, pool, table, kv_len, Ks, Vs = build_case(rows, bl, lengths, seed=seed)
    q, pool, tab = q.to(dev), pool.to(dev), torch.from_numpy(table).to(dev)
    plan = AttnPlan(kv_len, bl, q.shape[2], dev, target_items=target, min_split_keys=min_split)
    out_ws = torch.empty(q.shape, dtype=torch.bfloat16, device=dev)
    plan.run(q, pool, tab, out_ws, 0.125)
    out_na = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device=dev)
    n_merge = 0 if plan.merge is None else int(plan.merge.shape[0])
    rc = noalloc_fn()(q.data_ptr(), pool.data_ptr(), pool.shape[0], tab.data_ptr(), tab.stride(0), tab.shape[1],
                      plan.kv_len.data_ptr(), rows, bl, q.shape[2], plan.work.data_ptr(), int(plan.work.shape[0]),
                      kernels.ptr(plan.merge), n_merge, None, int(plan.n_slots), 0.125, 0, out_na.data_ptr(),
                      kernels.stream_ptr(dev))
    kernels.check(rc)
    torch.cuda.synchronize()
    return out_ws.cpu(), out_na.cpu(), plan, reference(q.cpu(), Ks, Vs)


def test_noalloc_equals_workspace_entry_two_calls(dev):
    a_ws, a_na, plan_a, ref_a = run_pair(dev, 4, 32, [1500, 33, 700, 2000], seed=31, target=64, min_split=32)
    assert plan_a.n_slots > 8  # split items wrote partials into the static array
    b_ws, b_na, plan_b, ref_b = run_pair(dev, 2, 16, [900, 300], seed=32, target=16, min_split=32)
    assert 0 < plan_b.n_slots < plan_a.n_slots
    assert torch.equal(a_na, a_ws) and torch.equal(b_na, b_ws)
    assert (a_na.float() - ref_a).abs().max().item() <= 2e-2
    assert (b_na.float() - ref_b).abs().max().item() <= 2e-2


def test_noalloc_unsplit_plan(dev):
    ws, na, plan, ref = run_pair(dev, 3, 32, [100, 200, 300], seed=33, target=1024, min_split=1024)
    assert plan.n_slots == 0
    assert torch.equal(na, ws)


def test_noalloc_rejects_partials_beyond_the_static_array(dev):
    q = torch.zeros(1, 64, 16, 64, dtype=torch.bfloat16, device=dev)
    pool = torch.zeros(4, 2, 16, 1024, dtype=torch.bfloat16, device=dev)
    tab = torch.zeros(1, 4, dtype=torch.int32, device=dev)
    kvl = torch.full((1,), 64, dtype=torch.int32, device=dev)
    work = torch.tensor([[0, 0, 64, 0]], dtype=torch.int32, device=dev)
    merge = torch.tensor([[0, 0, 1]], dtype=torch.int32, device=dev)
    out = torch.zeros_like(q)
    # 64 x 16 x 66 x 4 B = 270,336 B per slot: 62 slots fit in 16 MiB, 64 do not
    rc = noalloc_fn()(q.data_ptr(), pool.data_ptr(), 4, tab.data_ptr(), 4, 4, kvl.data_ptr(), 1, 64, 16,
                      work.data_ptr(), 1, merge.data_ptr(), 1, None, 64, 0.125, 0, out.data_ptr(),
                      kernels.stream_ptr(dev))
    assert rc == 1
    assert "static scratch holds" in kernels.load_library().yapd_last_error().decode()


def test_noalloc_under_graph_capture_equals_eager(dev):
    """The entry point captured in a HIP graph (torch.cuda.CUDAGraph) and replayed three times, with
    eager calls of the workspace entry point between the replays, equals the eager call bit for bit
    (the static array's address was looked up by an earlier call on this device)."""
    rows, bl = 4, 32
    q, pool, table, kv_len, Ks, Vs = build_case(rows, bl, [1500, 33, 700, 2000], seed=34)
    q, pool, tab = q.to(dev), pool.to(dev), torch.from_numpy(table).to(dev)
    plan = AttnPlan(kv_len, bl, q.shape[2], dev, target_items=64, min_split_keys=32)
    assert plan.n_slots > 0
    eager = torch.empty(q.shape, dtype=torch.bfloat16, device=dev)
    plan.run(q, pool, tab, eager, 0.125)
    out = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device=dev)
    n_merge = int(plan.merge.shape[0])

    def call():
        kernels.check(noalloc_fn()(q.data_ptr(), pool.data_ptr(), pool.shape[0], tab.data_ptr(), tab.stride(0),
                                   tab.shape[1], plan.kv_len.data_ptr(), rows, bl, q.shape[2],
                                   plan.work.data_ptr(), int(plan.work.shape[0]), plan.merge.data_ptr(), n_merge,
                                   None, int(plan.n_slots), 0.125, 0, out.data_ptr(), kernels.stream_ptr(dev)))
    call()  # eager, outside the capture
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for rep in range(3):
        out.fill_(float("nan"))
        scratch_other = torch.empty_like(eager)
        plan.run(q, pool, tab, scratch_other, 0.125)  # eager work between the replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep


def test_noalloc_first_call_under_capture_in_a_fresh_process(dev):
    """In a new process, the first call of the entry point runs inside a graph capture, so the
    scratch address is looked up during the capture (in relaxed capture mode); the replays must
    equal the eager workspace entry point (tests/_noalloc_capture_child.py)."""
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_noalloc_capture_child.py")
    res = subprocess.run([sys.executable, child], capture_output=True, text=True, timeout=180)
    assert res.returncode == 0 and "OK" in res.stdout, res.stdout[-2000:] + res.stderr[-2000:]
