"""GPU numerics of the bf16 MFMA GEMM family (b) and the RMSNorm rows against
plain PyTorch fp32 references with the reference's bf16 rounding points
(engines/flashinfer.py:433-455, 970-1065; HF LlamaRMSNorm, apply_rotary_pos_emb)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import llama as OL
from oracle import pages as OP
from yapd_amd import kernels

pytestmark = pytest.mark.gpu


def rnd(*shape, std=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).bfloat16()


def rel_err(out, ref):
    return ((out.float() - ref.float()).abs().max() / ref.float().abs().max().clamp_min(1e-6)).item()


# (16384 // 8, 8192, 1024), (2000, 8192, 1024), (4100, 4096, 2048) take the large-tile (256 x 256)
# path: >= 256 output tiles, M not a multiple of 256 in two of them.  M = 3072, N = 1024 is a grid of
# one 128 x 128 tile per CU, which runs three LDS stages: K = 64 / 128 / 192 give one, two and three
# k-tiles (the stage hand-off's short and tail cases); (3000, 1000, 4096) a ragged grid of that kind.
# Grids of at least two 256 x 256 tiles per CU take the persistent kernel: (4100, 8192, 1024) with a
# partial last row tile, (8000, 4196, 128) with a 100-column last tile and the shortest K it takes (two
# 64-wide k-tiles: no steady-state iteration), (8192, 8194, 192) with the 2-column tail split off to its
# own launch and three k-tiles (one steady-state iteration, no loads of a fourth).
@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (200, 3072, 1024), (1024, 1024, 4096), (37, 8194, 1024),
                                   (16384 // 8, 8192, 1024), (2000, 8192, 1024), (4100, 4096, 2048),
                                   (3072, 1024, 64), (3072, 1024, 128), (3072, 1024, 192), (3000, 1000, 4096),
                                   (4100, 8192, 1024), (8000, 4196, 128), (8192, 8194, 192)])
def test_gemm_bf16(dev, M, N, K):
    A = rnd(M, K, seed=1)
    W = rnd(N, K, std=0.02, seed=2)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    kernels.gemm_bf16(A.to(dev), W.to(dev), out)
    ref = A.to(dev).float() @ W.to(dev).float().T
    assert rel_err(out, ref) <= 8e-3


# (16384, 1000, 1024): persistent kernel, one round in XCD bands, a partial last column tile;
# (32768, 1024, 1024): persistent kernel, two rounds in row-major order; (16484, 1024, 1024): the
# same with 65 row tiles (no bands) and a partial last row tile
@pytest.mark.parametrize("M,N,K", [(200, 1024, 1024), (16384 // 8, 1024, 4096), (4100, 1024, 1024),
                                   (16384, 1000, 1024), (32768, 1024, 1024), (16484, 1024, 1024)])
def test_gemm_residual_equals_separate_add(dev, M, N, K):
    """The fused residual add is bit-identical to the projection stored in bf16
    followed by the bf16 residual add (HF's two roundings)."""
    A = rnd(M, K, seed=21).to(dev)
    W = rnd(N, K, std=0.02, seed=22).to(dev)
    res0 = rnd(M, N, seed=23).to(dev) * 4
    delta = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    kernels.gemm_bf16(A, W, delta)
    res = res0.clone()
    kernels.gemm_bf16_residual(A, W, res)
    assert torch.equal(res.cpu(), (res0 + delta).cpu())


def test_gemm_padded_ldc_and_strided_a(dev):
    M, N, K = 96, 300, 256
    base = rnd(M, K + 64, seed=3).to(dev)
    A = base[:, 32: 32 + K]
    W = rnd(N, K, std=0.05, seed=4).to(dev)
    out_full = torch.zeros(M, 312, dtype=torch.bfloat16, device=dev)
    out = out_full[:, :N]
    kernels.gemm_bf16(A, W, out)
    ref = A.float().cpu() @ W.float().cpu().T
    assert rel_err(out.cpu(), ref) <= 8e-3
    assert torch.count_nonzero(out_full[:, N:]) == 0  # nothing written past N


@pytest.mark.parametrize("M,K,Fd", [(300, 1024, 4096), (2000, 1024, 4096),  # 2000: large tiles, one round
                                     (4100, 1024, 4096), (4100, 256, 4096),  # persistent; ragged M; K < 16 k-tiles
                                     (8192, 1024, 1088),  # large tiles, the last one half past 2F
                                     (16384, 1024, 1088)])  # persistent, the last column tile half past 2F
def test_gemm_swiglu(dev, M, K, Fd):
    A = rnd(M, K, seed=5)
    Wg = rnd(Fd, K, std=0.02, seed=6)
    Wu = rnd(Fd, K, std=0.02, seed=7)
    act = torch.empty(M, Fd, dtype=torch.bfloat16, device=dev)
    kernels.gemm_swiglu(A.to(dev), kernels.interleave_gate_up(Wg, Wu).to(dev), act)
    A, Wg, Wu = A.to(dev), Wg.to(dev), Wu.to(dev)
    g = (A.float() @ Wg.float().T).bfloat16()
    u = (A.float() @ Wu.float().T).bfloat16()
    ref = (F.silu(g.float()).bfloat16().float() * u.float()).bfloat16()
    assert rel_err(act, ref.float()) <= 1.5e-2


# 70 x 32 rows: large tiles; 64 x 32: the 2 last columns split off; 300 x 32 and 512 x 32 (the step's
# shape): the persistent kernel and the split-off tail, 300 x 32 with a partial last row tile
@pytest.mark.parametrize("rows", [6, 70, 64, 300, 512])
def test_gemm_head_shift(dev, rows):
    bl, D, V = 32, 1024, 8194
    hidden = rnd(rows, bl, D, seed=8)
    ctx = rnd(rows, 1, D, seed=9)
    W = rnd(V, D, std=0.02, seed=10)
    logits = torch.empty(rows, bl, 8200, dtype=torch.bfloat16, device=dev)[..., :V]
    kernels.gemm_head_shift(hidden.to(dev), ctx.to(dev), W.to(dev), logits)
    ref = OL.speech_head_shift(hidden.to(dev).float(), ctx.to(dev).float(), W.to(dev).float())
    assert rel_err(logits, ref) <= 8e-3


# 180 x 32 rows: large-tile path.  6 heads at 320 x 32 rows: 256-column tiles
# straddle the q/k boundary (q = columns [0, 384)) and one tile holds only V
# columns (no RoPE rows staged); 2 heads: q, k and v inside one small tile.
# 512 x 32 rows (the step's shape) and 515 x 32: the persistent kernel, in XCD
# row bands and, with 65 row tiles (the last one partial), row-major; also at
# blocks of 16 (704 x 16 rows: 44 row tiles, row-major) and 64 (256 x 64
# rows), whose blocks start at any slot of a page like the others.
@pytest.mark.parametrize("rows,H,bl", [(3, 16, 32), (180, 16, 32), (320, 6, 32), (3, 2, 32), (512, 16, 32),
                                       (515, 16, 32), (704, 16, 16), (256, 16, 64)])
def test_gemm_qkv_rope_kv(dev, rows, H, bl):
    D = 1024
    M = rows * bl
    A = rnd(M, D, seed=11)
    Wqkv = rnd(3 * H * 64, D, std=0.02, seed=12)
    pos0 = [7, 150, 600] if rows == 3 else np.random.default_rng(1).integers(0, 700, rows).tolist()
    # HF default RoPE table (theta 10000) in the model dtype, as the engine builds it
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2).float() / 64))
    t = torch.arange(1024).float()
    fr = torch.outer(t, inv)
    emb = torch.cat([fr, fr], -1)
    cos_b, sin_b = emb.cos().bfloat16(), emb.sin().bfloat16()
    n_pages = rows * 48 + 16
    table = np.random.default_rng(0).permutation(n_pages)[: rows * 48].reshape(rows, 48).astype(np.int32)
    pool = torch.zeros(n_pages, 2, H, 1024, dtype=torch.bfloat16, device=dev)
    q_out = torch.empty(M, H * 64, dtype=torch.bfloat16, device=dev)
    kernels.gemm_qkv_rope_kv(A.to(dev), Wqkv.to(dev), cos_b.float().to(dev), sin_b.float().to(dev),
                             torch.tensor(pos0, dtype=torch.int32, device=dev), bl, q_out, pool,
                             torch.from_numpy(table).to(dev))
    qkv = (A.float() @ Wqkv.float().T).bfloat16()
    q = qkv[:, : H * 64].view(rows, bl, H, 64)
    k = qkv[:, H * 64: 2 * H * 64].view(rows, bl, H, 64)
    v = qkv[:, 2 * H * 64:].view(M, H, 64)
    pos = torch.stack([torch.arange(p, p + bl) for p in pos0])
    q = OL.rope(q, cos_b[pos], sin_b[pos])
    k = OL.rope(k, cos_b[pos], sin_b[pos]).reshape(M, H, 64)
    assert rel_err(q_out.cpu().view(rows, bl, H, 64), q.float()) <= 1.6e-2
    pool_ref = torch.zeros(n_pages, 2, H, 1024, dtype=torch.bfloat16)
    OP.pool_write(pool_ref, table, pos0, k, v)
    assert rel_err(pool.cpu(), pool_ref.float()) <= 1.6e-2
    # slots outside the block positions stay untouched
    touched = pool_ref.abs().sum(-1) > 0
    assert torch.count_nonzero(pool.cpu().float().abs().sum(-1)[~touched]) == 0


def test_gemm_rmsnorm_qkv_rope_kv_equals_the_two_steps(dev):
    """The composed entry point (input RMSNorm into a workspace, then QKV + RoPE + KV write) equals
    yapd_rmsnorm followed by yapd_gemm_qkv_rope_kv bit for bit: normed rows, q and the whole pool."""
    D, H, bl, rows = 1024, 16, 32, 40
    M = rows * bl
    x = rnd(M, D, seed=21).to(dev)
    ln_w = (torch.rand(D, generator=torch.Generator().manual_seed(22)) + 0.5).bfloat16().to(dev)
    Wqkv = rnd(3 * H * 64, D, std=0.02, seed=23).to(dev)
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2).float() / 64))
    fr = torch.outer(torch.arange(1024).float(), inv)
    emb = torch.cat([fr, fr], -1)
    cos_t, sin_t = emb.cos().bfloat16().float().to(dev), emb.sin().bfloat16().float().to(dev)
    pos0 = torch.tensor(np.random.default_rng(3).integers(0, 700, rows), dtype=torch.int32, device=dev)
    n_pages = rows * 48 + 16
    table = torch.from_numpy(np.random.default_rng(4).permutation(n_pages)[: rows * 48].reshape(rows, 48)
                             .astype(np.int32)).to(dev)
    outs = []
    for composed in (True, False):
        normed = torch.zeros(M, D, dtype=torch.bfloat16, device=dev)
        q_out = torch.zeros(M, H * 64, dtype=torch.bfloat16, device=dev)
        pool = torch.zeros(n_pages, 2, H, 1024, dtype=torch.bfloat16, device=dev)
        if composed:
            kernels.gemm_rmsnorm_qkv_rope_kv(x, ln_w, 1e-5, normed, Wqkv, cos_t, sin_t, pos0, bl, q_out, pool, table)
        else:
            kernels.rmsnorm(x, ln_w, 1e-5, normed)
            kernels.gemm_qkv_rope_kv(normed, Wqkv, cos_t, sin_t, pos0, bl, q_out, pool, table)
        torch.cuda.synchronize()
        outs.append((normed, q_out, pool))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert outs[0][1].abs().sum() > 0
    # a call the QKV checks reject (M not a multiple of bl) launches nothing, not even the norm
    normed = torch.full((M, D), 3.0, dtype=torch.bfloat16, device=dev)
    lib = kernels.load_library()
    rc = lib.yapd_gemm_rmsnorm_qkv_rope_kv(
        x.data_ptr(), ln_w.data_ptr(), 1e-5, normed.data_ptr(), Wqkv.data_ptr(), M, D, H, cos_t.data_ptr(),
        sin_t.data_ptr(), cos_t.shape[0], pos0.data_ptr(), 24, q_out.data_ptr(), pool.data_ptr(), n_pages,
        table.data_ptr(), table.stride(0), table.shape[1], kernels.stream_ptr(dev))
    torch.cuda.synchronize()
    assert rc == 1 and b"bad positions" in lib.yapd_last_error()
    assert bool((normed == 3.0).all())


@pytest.mark.parametrize("with_delta", [False, True])
@pytest.mark.parametrize("D", [1024, 512, 1536, 2048])  # one to four 512-wide chunks per row
def test_rmsnorm(dev, with_delta, D):
    M = 333
    x = rnd(M, D, seed=13) * 3
    w = (torch.rand(D, generator=torch.Generator().manual_seed(14)) + 0.5).bfloat16()
    delta = rnd(M, D, seed=15)
    out = torch.empty(M, D, dtype=torch.bfloat16, device=dev)
    xd = x.to(dev)
    if with_delta:
        kernels.rmsnorm(xd, w.to(dev), 1e-5, out, delta=delta.to(dev))
        res = x + delta  # bf16 add, as the decoder layer's residual
        assert torch.equal(xd.cpu(), res)
    else:
        kernels.rmsnorm(xd, w.to(dev), 1e-5, out)
        res = x
    ref = OL.rms_norm(res, w, 1e-5)
    diff = (out.cpu().float() - ref.float()).abs()
    ulp = ref.float().abs() * 2 ** -7 + 1e-6
    assert (diff <= ulp).all()
    assert (diff > 0).float().mean().item() < 0.01  # all but a few match bit for bit


@pytest.mark.parametrize("epi", ["store", "residual", "swiglu", "qkv"])
def test_rows_do_not_depend_on_batch_size(dev, epi):
    """A row is bit-identical whether it is computed in a large call (256 x 256
    direct-load tiles), a mid-sized one (128 x 128 direct-load tiles of 8 waves,
    three LDS stages when the grid has at most one tile per CU, else two) or a
    small one (one-wave 64 x 64 direct-load tiles): all issue the same MFMA over
    K in the same order.  Continuous batching relies on it -- a request's tokens
    must not depend on how many requests share its step.  The two mid sizes per
    epilogue select the 128 x 128 kernel with three and with two stages; every
    row of each call is compared with the large call."""
    H, D, bl = 16, 1024, 32
    big, small = 16384, 96
    mids = {"store": (4096, 6144), "residual": (4096, 6144), "swiglu": (512, 1024), "qkv": (1024, 2048)}[epi]
    sizes = (big, *mids, small)
    A = rnd(big, D, seed=31).to(dev)
    if epi in ("store", "residual", "swiglu"):
        N = 8192 if epi == "swiglu" else 1024
        W = rnd(N, D, std=0.02, seed=32).to(dev)
        R = rnd(big, N, seed=33).to(dev)
        outs = []
        for M in sizes:
            if epi == "store":
                C = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
                kernels.gemm_bf16(A[:M], W, C)
            elif epi == "residual":
                C = R[:M].clone()
                kernels.gemm_bf16_residual(A[:M], W, C)
            else:
                C = torch.empty(M, N // 2, dtype=torch.bfloat16, device=dev)
                kernels.gemm_swiglu(A[:M], W, C)
            outs.append(C.cpu())
        for M, out in zip(sizes[1:], outs[1:]):
            assert torch.equal(outs[0][:M], out), M
        return
    Wqkv = rnd(3 * H * 64, D, std=0.02, seed=34).to(dev)
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2).float() / 64))
    fr = torch.outer(torch.arange(1024).float(), inv)
    emb = torch.cat([fr, fr], -1)
    cos_t, sin_t = emb.cos().bfloat16().float().to(dev), emb.sin().bfloat16().float().to(dev)
    rows_big = big // bl
    pos0 = torch.from_numpy(np.random.default_rng(5).integers(0, 700, rows_big).astype(np.int32)).to(dev)
    n_pages = rows_big * 48
    table = torch.from_numpy(np.random.default_rng(6).permutation(n_pages).reshape(rows_big, 48).astype(np.int32)).to(dev)
    res = []
    for M in sizes:
        pool = torch.zeros(n_pages, 2, H, 1024, dtype=torch.bfloat16, device=dev)
        q_out = torch.empty(M, H * 64, dtype=torch.bfloat16, device=dev)
        kernels.gemm_qkv_rope_kv(A[:M], Wqkv, cos_t, sin_t, pos0[: M // bl], bl, q_out, pool, table[: M // bl])
        res.append((q_out.cpu(), pool))
    for M, (q, pool) in zip(sizes[1:], res[1:]):
        pages = table[: M // bl].reshape(-1).long()
        assert torch.equal(res[0][0][:M], q), M
        assert torch.equal(res[0][1][pages].cpu(), pool[pages].cpu()), M


def test_down_rows_do_not_depend_on_batch_size_or_tile_order(dev):
    """down_proj + residual (N = 1024, K = 4096) at the sizes whose grids take
    each tile order: M = 32768 and 24576 are multi-round grids of 256 x 256
    tiles in the columns-fastest XCD band order, M = 16384 a single round in the
    band order, M = 4096 the 128 x 128 kernel.  Every row of each smaller call
    equals the largest call's bit for bit."""
    N, K = 1024, 4096
    sizes = (32768, 24576, 16384, 4096)
    A = rnd(sizes[0], K, std=0.05, seed=51).to(dev)
    W = rnd(N, K, std=0.02, seed=52).to(dev)
    R = rnd(sizes[0], N, seed=53).to(dev)
    outs = []
    for M in sizes:
        C = R[:M].clone()
        kernels.gemm_bf16_residual(A[:M], W, C)
        outs.append(C.cpu())
    for M, out in zip(sizes[1:], outs[1:]):
        assert torch.equal(outs[0][:M], out), M
    ref = R[:256].cpu().float() + (A[:256].cpu().float() @ W.cpu().float().T).bfloat16().float()
    assert rel_err(outs[0][:256], ref) <= 8e-3


def test_narrow_last_column_tile_is_split_bit_identically(dev):
    """N = 32 x 256 + 2 (the speech head): when the 2-column tile would add a
    round of 256 x 256 tiles, those columns run as a second launch on 64 x 64
    tiles.  Rows must equal those of a small call (one launch on 64 x 64
    tiles) bit for bit, and the tail columns must match the fp32 product."""
    D, N = 1024, 8194
    A = rnd(16384, D, seed=41).to(dev)
    W = rnd(N, D, std=0.02, seed=42).to(dev)
    outs = []
    for M in (16384, 2048, 96):  # 2112 -> 9 rounds, 264 -> 2 rounds: split; 96 rows: one small launch
        C = torch.empty(M, 8200, dtype=torch.bfloat16, device=dev)[:, :N]
        kernels.gemm_bf16(A[:M], W, C)
        outs.append(C.cpu())
    assert torch.equal(outs[0][:96], outs[2])
    assert torch.equal(outs[1][:96], outs[2])
    assert torch.equal(outs[0][:2048], outs[1])
    ref = A[:2048].cpu().float() @ W[-2:].cpu().float().T
    assert rel_err(outs[1][:, -2:], ref) <= 8e-3
