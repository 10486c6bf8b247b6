"""GPU parity of the paged KV write/gather (bit-exact) and of the paged
block attention (a) against the oracle's fp32 SDPA over each row's
gathered keys (engines/flashinfer.py:1037-1039, engines/torch_sdpa.py:274-341)."""

import numpy as np
import pytest
import torch

from oracle import llama as OL
from oracle import pages as OP
from yapd_amd import kernels
from yapd_amd.paged import AttnPlan
from yapd_amd.synthetic import log_uniform_lengths

pytestmark = pytest.mark.gpu
H = 16


def random_table(rows, pages_per_row, n_pages, seed):
    perm = np.random.default_rng(seed).permutation(n_pages)[: rows * pages_per_row]
    return perm.reshape(rows, pages_per_row).astype(np.int32)


def test_kv_write_gather_bit_exact(dev):
    rows, bl, n_pages, ppr = 3, 16, 40, 8
    table = random_table(rows, ppr, n_pages, 0)
    starts = [5, 17, 96]
    g = torch.Generator().manual_seed(0)
    k = torch.randn(rows * bl, H, 64, generator=g).bfloat16()
    v = torch.randn(rows * bl, H, 64, generator=g).bfloat16()
    pool_ref = torch.randn(n_pages, 2, H, 1024, generator=g).bfloat16()
    pool = pool_ref.to(dev)
    OP.pool_write(pool_ref, table, starts, k, v)
    kernels.kv_write(k.to(dev), v.to(dev), pool, torch.from_numpy(table).to(dev),
                     torch.tensor(starts, dtype=torch.int32, device=dev), bl)
    torch.cuda.synchronize()
    assert torch.equal(pool.cpu(), pool_ref)
    for r in range(rows):
        kvl = starts[r] + bl
        kg, vg = kernels.kv_gather(pool, torch.from_numpy(table[r]).to(dev), kvl)
        kr, vr = OP.pool_gather(pool_ref, table[r], kvl)
        assert torch.equal(kg.cpu(), kr) and torch.equal(vg.cpu(), vr)
        assert torch.equal(kg.cpu()[starts[r]:], k[r * bl:(r + 1) * bl])


def test_kv_write_strided_views(dev):
    # K and V read straight out of a fused [tokens, 3*H*64] QKV buffer
    rows, bl, n_pages = 2, 32, 16
    table = random_table(rows, 8, n_pages, 1)
    qkv = torch.randn(rows * bl, 3 * H * 64).bfloat16()
    k = qkv[:, H * 64: 2 * H * 64].view(rows * bl, H, 64)
    v = qkv[:, 2 * H * 64:].view(rows * bl, H, 64)
    pool_ref = torch.zeros(n_pages, 2, H, 1024, dtype=torch.bfloat16)
    OP.pool_write(pool_ref, table, [0, 40], k, v)
    pool = torch.zeros_like(pool_ref, device=dev)
    qd = qkv.to(dev)
    kernels.kv_write(qd[:, H * 64: 2 * H * 64].view(rows * bl, H, 64), qd[:, 2 * H * 64:].view(rows * bl, H, 64),
                     pool, torch.from_numpy(table).to(dev), torch.tensor([0, 40], dtype=torch.int32, device=dev), bl)
    torch.cuda.synchronize()
    assert torch.equal(pool.cpu(), pool_ref)


def build_case(rows, bl, lengths, seed, n_pages=None, H=H):
    """Pool filled through the oracle's scatter; returns everything the kernel needs."""
    g = torch.Generator().manual_seed(seed)
    kv_len = [L + bl for L in lengths]
    ppr = max((x + 15) // 16 for x in kv_len)
    n_pages = n_pages or rows * ppr + 7
    table = random_table(rows, ppr, n_pages, seed)
    pool = torch.zeros(n_pages, 2, H, 1024, dtype=torch.bfloat16)
    Ks, Vs = [], []
    for r in range(rows):
        K = torch.randn(kv_len[r], H, 64, generator=g).bfloat16()
        V = torch.randn(kv_len[r], H, 64, generator=g).bfloat16()
        OP.pool_write(pool, table[r: r + 1], [0], K, V)  # whole row as one "block"
        Ks.append(K)
        Vs.append(V)
    q = torch.randn(rows, bl, H, 64, generator=g).bfloat16()
    return q, pool, table, kv_len, Ks, Vs


def reference(q, Ks, Vs):
    out = []
    for r in range(q.shape[0]):
        o = OL._sdpa(q[r].float(), Ks[r].float(), Vs[r].float(), causal=False)
        out.append(o.view(q.shape[1], q.shape[2], 64))
    return torch.stack(out)


def run_gpu(dev, q, pool, table, kv_len, target_items, min_split_keys=128):
    plan = AttnPlan(kv_len, q.shape[1], q.shape[2], dev, target_items=target_items, min_split_keys=min_split_keys)
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=dev)
    plan.run(q.to(dev), pool.to(dev), torch.from_numpy(table).to(dev), out, 0.125)
    torch.cuda.synchronize()
    return out.cpu(), plan


@pytest.mark.parametrize("bl", [16, 32, 7, 64])
@pytest.mark.parametrize("split", [False, True])
def test_attention_matches_oracle(dev, bl, split):
    rows = 6
    lengths = log_uniform_lengths(rows, 64, 700, seed=bl)
    q, pool, table, kv_len, Ks, Vs = build_case(rows, bl, lengths, seed=bl + int(split))
    out, plan = run_gpu(dev, q, pool, table, kv_len, 4096 if split else 1024, 32 if split else 128)
    if split:
        assert plan.n_slots > 0  # the split-KV merge path ran
    ref = reference(q, Ks, Vs)
    err = (out.float() - ref).abs().max().item()
    assert err <= 2e-2, err


@pytest.mark.parametrize("heads", [4, 8])  # one and two four-head workgroups per item
@pytest.mark.parametrize("split", [False, True])
def test_attention_head_counts(dev, heads, split):
    rows, bl = 5, 16
    lengths = log_uniform_lengths(rows, 64, 700, seed=heads)
    q, pool, table, kv_len, Ks, Vs = build_case(rows, bl, lengths, seed=heads + int(split), H=heads)
    out, plan = run_gpu(dev, q, pool, table, kv_len, 4096 if split else 1024, 32 if split else 128)
    if split:
        assert plan.n_slots > 0  # the split-KV merge path ran
    err = (out.float() - reference(q, Ks, Vs)).abs().max().item()
    assert err <= 2e-2, err


def test_split_and_unsplit_agree(dev):
    rows, bl = 4, 32
    lengths = [1500, 33, 700, 2000]
    q, pool, table, kv_len, Ks, Vs = build_case(rows, bl, lengths, seed=3)
    a, _ = run_gpu(dev, q, pool, table, kv_len, 1024)
    b, plan = run_gpu(dev, q, pool, table, kv_len, 4096, 32)
    assert plan.n_slots > 0
    assert (a.float() - b.float()).abs().max().item() <= 1.6e-2


def test_garbage_beyond_kv_len_is_ignored(dev):
    rows, bl = 3, 16
    lengths = [20, 45, 130]
    q, pool, table, kv_len, Ks, Vs = build_case(rows, bl, lengths, seed=4)
    # poison every slot past each row's kv_len with NaN (K and V planes)
    for r in range(rows):
        for pos in range(kv_len[r], table.shape[1] * 16):
            p = int(table[r][pos // 16])
            pool[p, 0].view(H, 16, 64)[:, pos % 16] = float("nan")
            pool[p, 1].view(H, 64, 16)[:, :, pos % 16] = float("nan")
    out, _ = run_gpu(dev, q, pool, table, kv_len, 1024)
    assert torch.isfinite(out.float()).all()
    assert (out.float() - reference(q, Ks, Vs)).abs().max().item() <= 2e-2


def test_ragged_stress_shape(dev):
    # 256 sequences, prefixes log-uniform in [64, 2048], 16-token pages drawn at
    # random from a 65,536-page pool, block 16 (one layer of the stress test).
    rows, bl = 256, 16
    lengths = log_uniform_lengths(rows, 64, 2048, seed=0)
    kv_len = [L + bl for L in lengths]
    ppr = max((x + 15) // 16 for x in kv_len)
    n_pages = 65536
    table = random_table(rows, ppr, n_pages, 0)
    gd = torch.Generator(device=dev).manual_seed(0)
    pool = torch.randn(n_pages, 2, H, 1024, generator=gd, device=dev, dtype=torch.bfloat16)
    q = torch.randn(rows, bl, H, 64, generator=gd, device=dev, dtype=torch.bfloat16)
    plan = AttnPlan(kv_len, bl, H, dev)
    out = torch.empty_like(q)
    tab = torch.from_numpy(table).to(dev)
    plan.run(q, pool, tab, out, 0.125)
    torch.cuda.synchronize()
    # spot-check a few rows against the gathered fp32 reference
    for r in (0, 17, 128, 255):
        K, V = kernels.kv_gather(pool, tab[r], kv_len[r])
        ref = OL._sdpa(q[r].float().cpu(), K.float().cpu(), V.float().cpu(), causal=False).view(bl, H, 64)
        assert (out[r].float().cpu() - ref).abs().max().item() <= 2e-2


def reference_causal(q, Ks, Vs, kv_len, bl):
    """Query i of a row's block sees keys < kv_len - bl + i + 1 (prefix prefill)."""
    out = []
    for r in range(q.shape[0]):
        kvl = kv_len[r]
        mask = torch.arange(kvl)[None, :] <= (kvl - bl + torch.arange(bl))[:, None]
        s = torch.einsum("qhd,khd->hqk", q[r].float(), Ks[r].float()) * 0.125
        s = s.masked_fill(~mask[None], float("-inf"))
        o = torch.einsum("hqk,khd->qhd", s.softmax(-1), Vs[r].float())
        out.append(o)
    return torch.stack(out)


@pytest.mark.parametrize("bl", [16, 64])
def test_causal_split_items_shorter_than_the_block(dev, bl):
    """Causal attention split into 32-key items with kv_len % 32 != 0: the last
    item is shorter than the block, so the first queries see none of its keys
    (their partial has m = -inf, l = 0); the merge must skip it, not turn it
    into NaN."""
    rows = 3
    lengths = [5 + 64, 5 + 160, 21 + 320]  # kv_len % 32 = 5, 5, 21 (plus bl, a multiple of 16)
    q, pool, table, kv_len, Ks, Vs = build_case(rows, bl, lengths, seed=40 + bl)
    assert all(k % 32 not in (0,) for k in kv_len)
    plan = AttnPlan(kv_len, bl, H, dev, target_items=4096, min_split_keys=32)
    assert plan.n_slots > 0
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=dev)
    plan.run(q.to(dev), pool.to(dev), torch.from_numpy(table).to(dev), out, 0.125, causal=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    err = (out.cpu().float() - reference_causal(q, Ks, Vs, kv_len, bl)).abs().max().item()
    assert err <= 2e-2, err


def test_plan_longer_than_device_kv_len(dev):
    """The serving engine plans from upper bounds of the cache length and the
    kernel masks by the true device length: items wholly past it see no key."""
    rows, bl = 3, 16
    lengths = [40, 300, 1100]
    q, pool, table, kv_len, Ks, Vs = build_case(rows, bl, lengths, seed=44)
    slack = [200, 64, 40]  # the first row's last items lie entirely past its true length
    plan = AttnPlan([k + s for k, s in zip(kv_len, slack)], bl, H, dev, target_items=4096, min_split_keys=32)
    assert plan.n_slots > 0
    kv_dev = torch.tensor(kv_len, dtype=torch.int32, device=dev)
    ppr = max((k + s + 15) // 16 for k, s in zip(kv_len, slack))
    tab = torch.zeros(rows, ppr, dtype=torch.int32)
    tab[:, : table.shape[1]] = torch.from_numpy(table)
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=dev)
    kernels.attn_paged_block(q.to(dev), pool.to(dev), tab.to(dev), kv_dev, plan.work, plan.merge, plan.part_o,
                             plan.part_ml, out, 0.125)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert (out.cpu().float() - reference(q, Ks, Vs)).abs().max().item() <= 2e-2
