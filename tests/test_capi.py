"""The C-ABI library loads on a CPU-only host, exports every function that
include/*.h declares, and rejects bad arguments before any launch."""

import ctypes
import re
from pathlib import Path

import pytest

from yapd_amd import kernels

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(yapd_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    assert "yapd_score_cfg_pmi_unmask" in names and "yapd_last_error" in names


def test_library_exports_every_declared_symbol():
    lib = kernels.load_library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_library_exports_only_the_declared_c_abi():
    """The dynamic symbol table holds the declared yapd_* functions and no internal C++ helper."""
    import shutil
    import subprocess
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    lib_path = kernels.load_library()._name
    out = subprocess.run([nm, "-D", "--defined-only", lib_path], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert exported == set(declared_functions()), sorted(exported ^ set(declared_functions()))


def test_ctypes_signatures_cover_header():
    assert set(declared_functions()) <= set(kernels._SIGNATURES)


def test_abi_version_and_empty_error():
    lib = kernels.load_library()
    assert lib.yapd_abi_version() == 4  # the layouts of yapd_t3_layer and yapd_t3_workspace in include/yapd_t3.h
    assert isinstance(lib.yapd_last_error(), bytes)


def test_score_rejects_bad_arguments_without_launch():
    lib = kernels.load_library()
    fn = lib.yapd_score_cfg_pmi_unmask
    nul = None
    # bl = 0 is invalid; every pointer NULL: validation fails first, no GPU call.
    rc = fn(nul, 8194, 8194, 1, 0, 8194, 0, 1, 0, 0, nul, nul, nul, nul, nul, nul, 10, 0.5, 1, 8194, 6562,
            0.0, 0, 0, 0, nul, nul, nul, nul, nul, nul, nul)
    assert rc == 1
    rc = fn(ctypes.c_void_p(16), 8194, 8194, 1, 65, 8194, 0, 1, 0, 0, nul, nul, nul, nul, nul, nul, 10, 0.5, 1,
            8194, 6562, 0.0, 0, 0, 0, nul, nul, nul, nul, nul, nul, nul)
    assert rc == 1 and b"bl" in lib.yapd_last_error()
    with pytest.raises(ValueError):
        kernels.check(1)


# Device pointers are never dereferenced by the host-side checks, so a fake
# 16-byte-aligned address stands in for them; a rejected call returns
# YAPD_EINVAL before any HIP call, which is why these run without a GPU.
P = 4096
EINVAL = 1
GEMM = (P, 1024, P, 1024)
REJECTS = [
    ("yapd_gemm_bf16", (*GEMM, 0, 1024, 1024, P, 1024, None), b"need M, N >= 1"),
    ("yapd_gemm_bf16", (*GEMM, 64, 1024, 100, P, 1024, None), b"K=100"),
    ("yapd_gemm_bf16", (P + 2, 1024, P, 1024, 64, 1024, 1024, P, 1024, None), b"A must be 16-byte aligned"),
    ("yapd_gemm_bf16", (*GEMM, 64, 1024, 1024, P, 512, None), b"bad C"),
    ("yapd_gemm_bf16_residual", (*GEMM, 64, 1024, 1024, None, 1024, None), b"bad residual"),
    ("yapd_gemm_swiglu", (P, 1024, P, 64, 100, 1024, P, 100, None), b"F must be a multiple of 64"),
    ("yapd_gemm_head_shift", (P, None, 4, 32, 1024, P, 1024, 8194, P, 8200, None), b"bad shift_ctx"),
    ("yapd_gemm_qkv_rope_kv", (P, 1024, P, 48, 1024, 16, P, P, 2048, P, 32, P, P, 64, P, 8, 8, None),
     b"bad positions / table shape"),
    ("yapd_gemm_qkv_rope_kv", (P, 1024, P, 64, 1024, 16, P + 4, P, 2048, P, 32, P, P, 64, P, 8, 8, None),
     b"cos/sin must be 16-byte aligned"),
    ("yapd_gemm_rmsnorm_qkv_rope_kv", (P, None, 1e-5, P, P, 64, 1024, 16, P, P, 2048, P, 32, P, P, 64, P, 8, 8, None),
     b"rmsnorm: NULL pointer"),
    ("yapd_gemm_rmsnorm_qkv_rope_kv", (P, P, 1e-5, P, P, 64, 1000, 16, P, P, 2048, P, 32, P, P, 64, P, 8, 8, None),
     b"D must be a multiple of 512"),
    ("yapd_gemm_rmsnorm_qkv_rope_kv", (P, P, 1e-5, P, P, 48, 1024, 16, P, P, 2048, P, 32, P, P, 64, P, 8, 8, None),
     b"bad positions / table shape"),
    ("yapd_rmsnorm", (None, None, P, P, 1e-5, 64, 1000, P, None), b"D must be a multiple of 512"),
    ("yapd_rmsnorm", (P, P, P, P, 1e-5, 64, 1024, P, None), b"not both"),
    ("yapd_rmsnorm", (None, None, P, P, 1e-5, 0, 1024, P, None), b"empty"),
    ("yapd_qgemm_affine", (P, 1024, P, P, P, 3, 64, 64, 1024, 1024, P, 1024, None), b"bits must be 4 or 8"),
    ("yapd_qgemm_affine", (P, 1024, P, P, P, 4, 32, 64, 1024, 1024, P, 1024, None), b"group_size must be 64"),
    ("yapd_dequant_affine", (P, P, P, 3, 64, 1024, 1024, P, None), b"bits must be 4 or 8"),
    ("yapd_dequant_affine", (P, P, P, 4, 32, 1024, 1024, P, None), b"group_size must be 64"),
    ("yapd_dequant_affine", (P, P, P, 4, 64, 1024, 1000, P, None), b"K % 64 == 0"),
    ("yapd_dequant_affine", (P, P, P, 8, 64, 1024, 1024, P + 4, None), b"outputs must be non-NULL and 16-byte"),
    ("yapd_attn_paged_block", (P, P, 64, P, 8, 8, P, 4, 65, 16, P, 4, None, 0, None, None, None, 0, 0.125, 0, P,
                               None), b"1 <= bl <= 64"),
    ("yapd_attn_paged_block", (P, P, 64, P, 8, 8, P, 4, 32, 6, P, 4, None, 0, None, None, None, 0, 0.125, 0, P,
                               None), b"n_heads must be a multiple of 4"),
    ("yapd_attn_paged_block", (P, P, 64, P, 8, 8, P, 4, 32, 16, P, 4, P, 2, None, None, None, 0, 0.125, 0, P,
                               None), b"split items need a workspace"),
    ("yapd_kv_write", (P, P, 1028, 1028, P, 64, P, 8, 8, P, 4, 32, 16, None), b"multiples of 8"),
    ("yapd_kv_write", (P, P, 1024, 1024, P, 64, P, 8, 8, P, 0, 32, 16, None), b"empty shape"),
    ("yapd_kv_gather", (P, 64, None, 8, 100, 16, P, P, None), b"NULL pointer"),
    ("yapd_tick_update", (4, 16, 3, 1024, 10, 8194, 6562, 4096, 2048, P, 2048, P, P, P, P, P, P, P, P, P, P, P,
                          None), b"bad sizes"),
    ("yapd_tick_update", (4, 16, 2, 1024, 10, 8194, 6562, 16, 2048, P, 2048, P, P, P, P, P, P, P, P, P, P, P,
                          None), b"bad max_len"),
    ("yapd_snake", (P, P, None, P, 2, 64, 0, None), b"need B, C, T >= 1"),
    ("yapd_residual_bias", (P, None, P, P, 2, 64, 100, None), b"NULL residual"),
    ("yapd_mean3", (P, P, P, P, 0, None), b"n must be >= 1"),
    ("yapd_residual_bias_snake", (P, P, P, None, P, P, 2, 64, 100, None), b"NULL pointer"),
    ("yapd_branch_start", (P, P, P, P, P, P, P, None, P, 2, 64, 100, None), b"NULL pointer"),
    ("yapd_voc_stitch", (P, 960, 960, 2, P, 70000, P, P, 480, P, 960, None, 0, None, 0, P, 100, None),
     b"n_jobs must be in [0, 65535]"),
    ("yapd_voc_stitch", (P, 100, 960, 2, P, 3, P, P, 480, P, 960, None, 0, None, 0, P, 100, None), b"bad wav shape"),
    ("yapd_voc_stitch", (P, 960, 960, 2, P, 3, P, None, 480, P, 960, None, 0, None, 0, P, 100, None),
     b"both fade ramps"),
    ("yapd_voc_stitch", (P, 960, 960, 2, P, 3, P, P, 480, P, 960, None, 2, None, 0, P, 100, None), b"NULL tails_in"),
    ("yapd_voc_stitch", (P, 960, 960, 2, P, 3, P, P, 480, None, 960, None, 0, None, 0, P, 100, None), b"NULL trim"),
    ("yapd_mfma_peak_probe", (0, 10, 1, P, None), b"1 <= blocks"),
    ("yapd_hbm_read_probe", (P, 100, 8, P, None), b"multiple of 16"),
    ("yapd_hbm_read_probe", (P + 4, 1024, 8, P, None), b"16-byte aligned"),
]


@pytest.mark.parametrize("name,args,msg", REJECTS, ids=[f"{r[0]}-{i}" for i, r in enumerate(REJECTS)])
def test_entry_points_reject_bad_arguments_without_launch(name, args, msg):
    lib = kernels.load_library()
    assert getattr(lib, name)(*args) == EINVAL
    assert msg in lib.yapd_last_error(), lib.yapd_last_error()


def test_tick_update_with_no_slots_is_a_no_op():
    lib = kernels.load_library()
    assert lib.yapd_tick_update(0, 16, 2, 1024, 10, 8194, 6562, 4096, 2048, None, 2048, *([None] * 11), None) == 0


def _block_forward_args(**model_overrides):
    layer = kernels.T3Layer(P, P, P, P, P, P, 1e-5, 1e-5, P)
    layers = (kernels.T3Layer * 2)(layer, layer)
    fields = dict(n_layers=2, hidden=1024, n_heads=16, ffn=4096, layers=layers, final_norm=P, final_eps=1e-5,
                  rope_cos=P, rope_sin=P, rope_positions=2048, n_pages=64, page_table=P, table_stride=8,
                  table_cols=8)
    fields.update(model_overrides)
    model = kernels.T3Model(**fields)
    ws = kernels.T3Workspace(P, P, P, P, P, P, P, 4, None, 0, None, None, None, 0)
    return model, ws, layers


@pytest.mark.parametrize("override,msg", [
    (dict(n_heads=6), b"n_heads must be a multiple of 4"),
    (dict(ffn=100), b"ffn must be a multiple of 64"),
    (dict(hidden=1000), b"hidden must be"),
    (dict(rope_cos=None), b"missing RoPE tables"),
    (dict(table_stride=4), b"bad page table"),
])
def test_block_forward_checks_every_layer_rule_before_launching(override, msg):
    """A shape that only a later per-layer call would reject is refused before
    the first launch, so nothing (residual, KV pools, outputs) is modified."""
    lib = kernels.load_library()
    model, ws, _keep = _block_forward_args(**override)
    rc = lib.yapd_t3_block_forward(ctypes.byref(model), ctypes.byref(ws), P, 4, 32, P, P, 0, P, None, 0, None,
                                   None, 0, None)
    assert rc == EINVAL and msg in lib.yapd_last_error(), lib.yapd_last_error()


@pytest.mark.parametrize("n_tokens,rows,max_q,msg", [
    (0, 4, 64, b"n_tokens"), (300, 4, 64, b"n_tokens <= rows * max_q"), (10, 4, 65, b"max_q <= 64"),
    (10, 0, 64, b"rows >= 1")])
def test_packed_prefill_checks_before_launching(n_tokens, rows, max_q, msg):
    lib = kernels.load_library()
    model, ws, _keep = _block_forward_args()
    rc = lib.yapd_t3_prefill_packed(ctypes.byref(model), ctypes.byref(ws), P, n_tokens, rows, max_q, P, P, P, P, P,
                                    None)
    assert rc == EINVAL and msg in lib.yapd_last_error(), lib.yapd_last_error()
    model, ws, _keep = _block_forward_args(n_heads=6)
    rc = lib.yapd_t3_prefill_packed(ctypes.byref(model), ctypes.byref(ws), P, 10, 4, 64, P, P, P, P, P, None)
    assert rc == EINVAL and b"n_heads must be a multiple of 4" in lib.yapd_last_error()
    rc = lib.yapd_t3_prefill_packed(ctypes.byref(model), ctypes.byref(ws), P, 10, 4, 64, None, P, P, P, P, None)
    assert rc == EINVAL and b"NULL pointer" in lib.yapd_last_error()


def test_block_forward_checks_alignment_and_quant_layers_before_launching():
    """Misaligned workspace or partials pointers and bad quantised layers are
    refused by the up-front checks (EINVAL here, where no launch could run:
    the checks come before any launch, so nothing is modified)."""
    lib = kernels.load_library()

    def call(model, ws):
        return lib.yapd_t3_block_forward(ctypes.byref(model), ctypes.byref(ws), P, 4, 32, P, P, 0, P, None, 0, None,
                                         None, 0, None)
    model, ws, _keep = _block_forward_args()
    ws.q = P + 4
    assert call(model, ws) == EINVAL and b"16-byte aligned" in lib.yapd_last_error()
    model, ws, _keep = _block_forward_args()
    ws.work = P + 8
    assert call(model, ws) == EINVAL and b"16-byte aligned" in lib.yapd_last_error()
    model, ws, _keep = _block_forward_args()
    ws.merge, ws.n_merge, ws.part_o, ws.part_ml, ws.n_slots = P, 2, P + 4, P, 4
    assert call(model, ws) == EINVAL and b"part_o must be 16-byte aligned" in lib.yapd_last_error()
    rc = lib.yapd_t3_prefill_packed(ctypes.byref(model), ctypes.byref(ws), P, 10, 4, 64, P, P, P, P, P, None)
    assert rc == EINVAL and b"part_o must be 16-byte aligned" in lib.yapd_last_error()
    model, ws, layers = _block_forward_args()
    layers[1].qbits = 3
    assert call(model, ws) == EINVAL and b"bits must be 4 or 8" in lib.yapd_last_error()
    layers[1].qbits = 4
    assert call(model, ws) == EINVAL and b"NULL quantised weight" in lib.yapd_last_error()
    # (never a fully valid layer set: these pointers are not device memory)
    for name in ("q_qkv", "q_o", "q_gate_up"):
        setattr(layers[1], name, kernels.T3QWeight(P, P, P))
    layers[1].w_qkv = None  # unused by a quantised layer: the next rule is the one reported
    layers[1].q_down = kernels.T3QWeight(P + 4, P, P)
    assert call(model, ws) == EINVAL and b"q_down: packed weights must be 16-byte aligned" in lib.yapd_last_error()
    # the dequantise-once scratch: one layer's four weights, 16-byte aligned
    layers[1].q_down = kernels.T3QWeight(P, P, P)
    need = 3 * 1024 * 1024 + 1024 * 1024 + 2 * 4096 * 1024 + 1024 * 4096
    ws.wdq, ws.wdq_elems = P, need - 8
    assert call(model, ws) == EINVAL and b"wdq must be 16-byte aligned and hold %d bf16" % need in lib.yapd_last_error()
    ws.wdq, ws.wdq_elems = P + 4, need
    assert call(model, ws) == EINVAL and b"wdq must be 16-byte aligned" in lib.yapd_last_error()


def test_block_forward_rejects_incomplete_layer_and_head():
    lib = kernels.load_library()
    model, ws, layers = _block_forward_args()
    layers[1].w_down = None
    rc = lib.yapd_t3_block_forward(ctypes.byref(model), ctypes.byref(ws), P, 4, 32, P, P, 0, P, None, 0, None,
                                   None, 0, None)
    assert rc == EINVAL and b"layer 1 has a NULL weight" in lib.yapd_last_error()
    model, ws, _keep = _block_forward_args()
    rc = lib.yapd_t3_block_forward(ctypes.byref(model), ctypes.byref(ws), P, 4, 32, P, P, 0, P, P, 8194, P,
                                   P, 8000, None)
    assert rc == EINVAL and b"ld_logits >= vocab" in lib.yapd_last_error()
