"""Child process of test_zz_no_alloc.py: the first ``yapd_attn_paged_block_noalloc`` call of this
process runs under HIP graph capture (so its scratch-address lookup happens inside the capture);
three replays must equal the workspace entry point's eager output bit for bit.  Prints OK."""

import os
import sys

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from test_gpu_attention import build_case  # noqa: E402
from yapd_amd import kernels  # noqa: E402
from yapd_amd.paged import AttnPlan  # noqa: E402


def main():
    dev = torch.device("cuda:0")
    lib = kernels.load_library()
    rows, bl = 4, 32
    q, pool, table, kv_len, _, _ = build_case(rows, bl, [1500, 33, 700, 2000], seed=35)
    q, pool, tab = q.to(dev), pool.to(dev), torch.from_numpy(table).to(dev)
    plan = AttnPlan(kv_len, bl, q.shape[2], dev, target_items=64, min_split_keys=32)
    eager = torch.empty(q.shape, dtype=torch.bfloat16, device=dev)
    plan.run(q, pool, tab, eager, 0.125)
    out = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.yapd_attn_paged_block_noalloc(
            q.data_ptr(), pool.data_ptr(), pool.shape[0], tab.data_ptr(), tab.stride(0), tab.shape[1],
            plan.kv_len.data_ptr(), rows, bl, q.shape[2], plan.work.data_ptr(), int(plan.work.shape[0]),
            plan.merge.data_ptr(), int(plan.merge.shape[0]), None, int(plan.n_slots), 0.125, 0, out.data_ptr(),
            kernels.stream_ptr(dev))
    kernels.check(rc)
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    print("OK", flush=True)


if __name__ == "__main__":
    main()
