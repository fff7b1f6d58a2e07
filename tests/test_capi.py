"""
The C-ABI boundary without a GPU: libnsmoe.so loads, exports every function that
include/nsmoe.h declares, agrees with the Python mirror on the layout of its argument
structs and on the dispatch size formulas, and rejects bad arguments with an error
string before launching anything.
"""

import ctypes
import re
from pathlib import Path

import pytest

from nanospeaker_amd import _native as nat
from nanospeaker_amd import moe_kernel as mk

HEADER = Path(__file__).resolve().parents[1] / "include" / "nsmoe.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(nsmoe_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = nat.lib()
    names = declared_functions()
    assert len(names) >= 16
    for name in names:
        assert hasattr(lib, name), f"{name} declared in nsmoe.h but not exported"
        assert name in nat.SIGNATURES, f"{name} has no ctypes signature"


def test_struct_layouts_match_the_header():
    # nsmoe_experts_args: 2 x i32, i64, 6 x i32, i64, then 15 pointers
    assert ctypes.sizeof(nat.ExpertsArgs) == 4 * 2 + 8 + 4 * 6 + 8 + 8 * 15
    assert nat.ExpertsArgs.x.offset == 48
    assert ctypes.sizeof(nat.ExpertsGrads) == 8 * 10
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = text[text.index("typedef struct nsmoe_experts_args"):text.index("} nsmoe_experts_args")]
    fields = re.findall(r"\b(\w+);", body)
    assert fields == [f for f, _ in nat.ExpertsArgs._fields_]


def test_attn_args_layout_matches_the_header():
    # nsmoe_attn_args: 4 x i32, 2 x i64, 2 x i32, f32, i32, then 6 pointers
    assert ctypes.sizeof(nat.AttnArgs) == 4 * 4 + 8 * 2 + 4 * 4 + 8 * 6
    assert nat.AttnArgs.qkv.offset == 48
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = text[text.index("typedef struct nsmoe_attn_args"):text.index("} nsmoe_attn_args")]
    assert re.findall(r"\b(\w+);", body) == [f for f, _ in nat.AttnArgs._fields_]


def _attn(**kw):
    base = dict(dtype=0, n_heads=9, n_kv_heads=3, head_dim=64, batch=1, seq_len=16,
                ld=960, window=0, eps=1e-6, reserved=0, qkv=16, q_gamma=16, k_gamma=16,
                cos=16, sin=16, out=16)
    base.update(kw)
    return nat.AttnArgs(**base)


@pytest.mark.parametrize("kw,needle", [
    (dict(dtype=2), "16-bit"),
    (dict(head_dim=128), "head_dim"),
    (dict(n_heads=9, n_kv_heads=2), "n_heads"),
    (dict(n_heads=10, n_kv_heads=2), "n_heads"),
    (dict(ld=900), "pitch"),
    (dict(window=-1), "window"),
    (dict(qkv=None), "NULL"),
    (dict(qkv=8), "misaligned"),
])
def test_attn_prefill_rejects_bad_arguments(kw, needle):
    lib = nat.lib()
    assert lib.nsmoe_attn_prefill(_attn(**kw), None) == 1
    assert needle in lib.nsmoe_last_error().decode()


def test_attn_prefill_of_nothing_is_a_no_op():
    assert nat.lib().nsmoe_attn_prefill(_attn(batch=0, qkv=None), None) == 0
    assert nat.lib().nsmoe_attn_prefill(_attn(seq_len=0, qkv=None), None) == 0


@pytest.mark.parametrize("args,needle", [
    ((2, 16, 64, 4, 64, 16, -100, 16, 16, None), "16-bit"),
    ((0, 16, 64, 4, 60, 16, -100, 16, 16, None), "multiple of 8"),
    ((0, 16, 64, 4, 65544, 16, -100, 16, 16, None), "at most"),
    ((0, 16, 32, 4, 64, 16, -100, 16, 16, None), "pitch"),
    ((0, 16, 64, 4, 64, None, -100, 16, 16, None), "NULL"),
    ((0, 16, 64, 4, 64, 16, -100, None, 16, 16), "NULL"),
    ((0, 8, 64, 4, 64, 16, -100, 16, 16, None), "aligned"),
])
def test_cross_entropy_rows_rejects_bad_arguments(args, needle):
    lib = nat.lib()
    assert lib.nsmoe_cross_entropy_rows(*args, None) == 1
    assert needle in lib.nsmoe_last_error().decode()


@pytest.mark.parametrize("args,needle", [
    ((2, 16, 16, 1e-6, 4, 64, 16, None), "16-bit"),
    ((0, 16, 16, 1e-6, 4, 60, 16, None), "d %"),
    ((0, 16, 16, 1e-6, 4, 2048, 16, None), "d %"),
    ((0, 16, 16, 1e-6, -1, 64, 16, None), "n_rows"),
    ((0, None, 16, 1e-6, 4, 64, 16, None), "NULL"),
    ((0, 8, 16, 1e-6, 4, 64, 16, None), "aligned"),
])
def test_rms_norm_rejects_bad_arguments(args, needle):
    lib = nat.lib()
    assert lib.nsmoe_rms_norm(*args, None) == 1
    assert needle in lib.nsmoe_last_error().decode()


def test_abi_version_and_alignment():
    assert nat.lib().nsmoe_abi_version() == nat.ABI_VERSION == 8
    assert nat.lib().nsmoe_align_m() == mk.ALIGN_M


@pytest.mark.parametrize("m,e", [(0, 8), (1, 8), (49152, 76), (384, 76), (100, 1000), (15, 8)])
def test_l_cap_matches_python(m, e):
    assert nat.lib().nsmoe_dispatch_l_cap(m, e) == mk._l_cap(m, e)


def test_workspace_sizes_are_positive_and_grow():
    a = nat.ExpertsArgs(dtype=0, activation=0, n_tokens=8192, d_model=576, d_hidden=128,
                        n_experts=76, n_shared=2, top_k=6, l_cap=mk._l_cap(49152, 76))
    fwd = nat.lib().nsmoe_experts_fwd_workspace_size(a)
    bwd = nat.lib().nsmoe_experts_bwd_workspace_size(a)
    assert fwd >= (49152 + 2 * 8192) * 576 * 2
    assert bwd > fwd
    # [chunks, E] int32 histograms; chunks of 1024 pairs while E <= 256, else 256
    assert nat.lib().nsmoe_dispatch_workspace_size(49152, 76) == 48 * 76 * 4
    assert nat.lib().nsmoe_dispatch_workspace_size(49152, 1000) == 192 * 1000 * 4


def test_pack_sizes_match_the_fragment_layout():
    a = nat.ExpertsArgs(dtype=0, activation=0, n_tokens=8192, d_model=576, d_hidden=128,
                        n_experts=76, n_shared=2, top_k=6, l_cap=mk._l_cap(49152, 76))
    nin, nout = ctypes.c_size_t(), ctypes.c_size_t()
    assert nat.lib().nsmoe_pack_sizes(a, ctypes.byref(nin), ctypes.byref(nout)) == 0
    frag = 64 * 8 * 2                      # one 16 x 32 bf16 fragment
    assert nin.value == 78 * 16 * 18 * frag  # 2 * 128 / 16 column blocks, 576 / 32 k blocks
    assert nout.value == 78 * 36 * 4 * frag  # 576 / 16 column blocks, 128 / 32 k blocks
    w_sh = torch_empty = None
    import torch
    x = torch.empty(8192, 576, dtype=torch.bfloat16)
    w_in = torch.empty(76, 576, 256, dtype=torch.bfloat16)
    w_sh_in = torch.empty(2, 576, 256, dtype=torch.bfloat16)
    assert mk._packed_in_bytes(x, w_in, w_sh_in) == nin.value


@pytest.mark.parametrize("call,needle", [
    (lambda L: L.nsmoe_route_fwd(None, 4, 0, 1, 0, 0, None, None, None, None), "n_experts"),
    (lambda L: L.nsmoe_route_fwd(None, 4, 300, 1, 0, 0, None, None, None, None), "n_experts"),
    (lambda L: L.nsmoe_route_fwd(None, 4, 8, 9, 0, 0, None, None, None, None), "top_k"),
    (lambda L: L.nsmoe_route_fwd(None, 4, 8, 2, 1, 0, None, None, None, None), "probs"),
    (lambda L: L.nsmoe_route_bwd(None, None, None, 0, None, None, None, 0.0, 4, 8, 0, 0, None,
                                 None), "top_k"),
    (lambda L: L.nsmoe_route_fwd(None, 4, 8, 2, 4, 2, None, None, None, None), "16-bit"),
    (lambda L: L.nsmoe_balance_loss(None, None, 4, 0, 0.01, None, None, 0, None), "n_experts"),
    (lambda L: L.nsmoe_balance_loss(None, None, 4, 8, 0.01, None, None, 0, None), "NULL"),
    (lambda L: L.nsmoe_dispatch(None, -1, 8, None, None, None, None, None, None, None, 0, None),
     "n_pairs"),
    (lambda L: L.nsmoe_dispatch(None, 10, 0, None, None, None, None, None, None, None, 0, None),
     "n_experts"),
])
def test_bad_arguments_are_rejected_with_a_message(call, needle):
    lib = nat.lib()
    rc = call(lib)
    assert rc == 1
    assert needle in lib.nsmoe_last_error().decode()


def test_dispatch_workspace_too_small_is_an_error():
    lib = nat.lib()
    rc = lib.nsmoe_dispatch(1, 100, 8, 1, 1, 1, 1, 1, 1, 1, 4, None)
    assert rc == 3 and "workspace" in lib.nsmoe_last_error().decode()


def test_experts_argument_validation():
    lib = nat.lib()
    bad = nat.ExpertsArgs(dtype=7, activation=0, n_tokens=1, d_model=8, d_hidden=8,
                          n_experts=2, n_shared=0, top_k=1, l_cap=16)
    assert lib.nsmoe_experts_fwd(bad, None, None, None, 0, None) == 1
    assert "dtype" in lib.nsmoe_last_error().decode()
    big = nat.ExpertsArgs(dtype=2, activation=0, n_tokens=1, d_model=8, d_hidden=200,
                          n_experts=2, n_shared=0, top_k=1, l_cap=16)
    assert lib.nsmoe_experts_fwd(big, None, None, None, 0, None) == 1
    assert "d_hidden" in lib.nsmoe_last_error().decode()
    empty = nat.ExpertsArgs(dtype=0, activation=0, n_tokens=0, d_model=8, d_hidden=8,
                            n_experts=2, n_shared=0, top_k=1, l_cap=0)
    assert lib.nsmoe_experts_fwd(empty, None, None, None, 0, None) == 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(nat, "_LIB", None)
    monkeypatch.setattr(nat, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(nat.NativeLibraryError):
        nat.lib()
    assert not nat.available()


def test_kernel_supported_raises_on_a_gpu_tensor_without_the_library(monkeypatch, tmp_path):
    """A GPU tensor never silently falls back: the missing build is an error."""
    class FakeCuda:
        is_cuda = True
        dtype = __import__("torch").bfloat16

    monkeypatch.setattr(nat, "_LIB", None)
    monkeypatch.setattr(nat, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(nat.NativeLibraryError):
        mk.kernel_supported(FakeCuda())


@pytest.mark.parametrize("n,e,k,dt,probs", [
    (8192, 76, 6, "bfloat16", True), (8192, 76, 6, "bfloat16", False), (1, 8, 2, "float32", True),
    (37, 76, 6, "float16", True), (32768, 76, 6, "bfloat16", False), (5, 1000, 8, "float32", False),
])
@pytest.mark.parametrize("save_act", [False, True])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("d,h,s", [(576, 128, 2), (64, 64, 0), (128, 64, 1), (192, 96, 2),
                                   (512, 256, 2), (320, 128, 2), (576, 48, 2)])
def test_block_saved_layout_matches_the_python_mirror(n, e, k, dt, probs, save_act, norm, d,
                                                      h, s):
    """The fake impl of nsmoe::block_fwd sizes `saved` in Python (symbolic shapes),
    including which shapes keep the experts' pre-activations, and the norm's parts."""
    import torch
    dtype = getattr(torch, dt)
    a = nat.ExpertsArgs(dtype=mk._DT[dtype], activation=0, n_tokens=n, d_model=d,
                        d_hidden=h, n_experts=e, n_shared=s, top_k=k, l_cap=0)
    offs = (ctypes.c_size_t * nat.BLOCK_NSAVED)()
    total = ctypes.c_size_t()
    flags = ((nat.ROUTE_PROBS if probs else 0) | (nat.BLOCK_SAVE_ACT if save_act else 0)
             | (nat.BLOCK_NORM if norm else 0))
    assert nat.lib().nsmoe_block_saved_layout(a, flags, offs, ctypes.byref(total)) == 0
    assert total.value == mk.block_saved_bytes(n, e, k, dtype, probs, save_act, d, h, s, norm)
    assert list(offs) == sorted(offs) and offs[0] == 0
    es = 4 if dtype == torch.float32 else 2
    assert offs[nat.SAVED_RSTD] - offs[nat.SAVED_XN] == (mk._al256(n * d * es) if norm else 0)
    assert total.value - offs[nat.SAVED_RSTD] == (mk._al256(n * 4) if norm else 0)
    act = offs[nat.SAVED_XN] - offs[nat.SAVED_ACT]
    if save_act and mk.save_act_supported(dtype, d, h):
        l_cap = mk._l_cap(n * k, e)
        assert act == mk._al256((l_cap + s * (-(-n // 16) * 16)) * 2 * h * 2)
    else:
        assert act == 0


def test_save_act_shapes():
    """The register-tiled kernels' shapes: nanoSpeaker's block takes them; fp32, H above
    128, d off the 64 grid and odd GEMM2 step counts do not."""
    import torch
    ok = mk.save_act_supported
    assert ok(torch.bfloat16, 576, 128) and ok(torch.float16, 576, 128)
    assert ok(torch.bfloat16, 128, 64) and ok(torch.bfloat16, 384, 96)
    assert not ok(torch.float32, 576, 128)
    assert not ok(torch.bfloat16, 576, 256) and not ok(torch.bfloat16, 576, 120)
    assert not ok(torch.bfloat16, 544, 128) and not ok(torch.bfloat16, 64, 64)
    assert not ok(torch.bfloat16, 192, 32)  # one pass x one k-step of H: odd


def test_tuning_options_round_trip_and_reject_bad_values():
    lib = nat.lib()
    for name, good, bad in (("side_stream", 1, 2), ("fwd_rows", 32, 80), ("bwd_rows", 96, 32),
                            ("dx_rows", 64, 48), ("fwd_dist", 6, 7), ("bwd_dist", 4, 5),
                            ("dx_dist", 4, 1), ("xcd_run", 8, 2048), ("dw_stages", 3, 5),
                            ("router_waves", 8, 4), ("pack_in_place", 1, 2)):
        assert nat.get_option(name) == 0
        nat.set_option(name, good)
        assert nat.get_option(name) == good
        assert lib.nsmoe_set_option(name.encode(), bad) == 1
        assert name in lib.nsmoe_last_error().decode()
        assert nat.get_option(name) == good
        nat.set_option(name, 0)
        assert nat.get_option(name) == 0
    assert lib.nsmoe_set_option(b"no_such_option", 1) == 1
    assert lib.nsmoe_get_option(b"no_such_option") == -1


def test_block_entry_points_reject_missing_buffers():
    lib = nat.lib()
    a = nat.ExpertsArgs(dtype=0, activation=0, n_tokens=4, d_model=64, d_hidden=64,
                        n_experts=8, n_shared=0, top_k=2, l_cap=0)
    #      args norm w_router bias logits flags coef saved idx counts out aux ws ws_bytes
    #      stream
    assert lib.nsmoe_block_fwd(a, None, None, None, 1, 0, 0.0, 1, None, 1, 1, None, 1,
                               1 << 20, None) == 1
    assert "NULL" in lib.nsmoe_last_error().decode()
    assert lib.nsmoe_block_fwd(a, None, None, None, 1, 0, 0.0, 1, 1, 1, 1, None, 1, 1 << 20,
                               None) == 1
    assert "packed" in lib.nsmoe_last_error().decode()
    a.w_in_packed = a.w_out_packed = 1
    assert lib.nsmoe_block_fwd(a, None, None, 1, 1, 0, 0.0, 1, 1, 1, 1, None, 1, 1 << 20,
                               None) == 1
    assert "logit_bias" in lib.nsmoe_last_error().decode()
    odd = nat.ExpertsArgs(dtype=0, activation=0, n_tokens=4, d_model=48, d_hidden=64,
                          n_experts=8, n_shared=0, top_k=2, l_cap=0, w_in_packed=1,
                          w_out_packed=1)
    assert lib.nsmoe_block_fwd(odd, None, 1, None, 1, 0, 0.0, 1, 1, 1, 1, None, 1, 1 << 20,
                               None) == 1
    assert "fused router" in lib.nsmoe_last_error().decode()
    # The norm and NSMOE_BLOCK_NORM go together, and the norm needs the fused router.
    norm = nat.BlockNorm(weight=1, grad_weight=1, eps=1e-6)
    assert lib.nsmoe_block_fwd(a, norm, 1, None, 1, 0, 0.0, 1, 1, 1, 1, None, 1, 1 << 20,
                               None) == 1
    assert "NSMOE_BLOCK_NORM" in lib.nsmoe_last_error().decode()
    assert lib.nsmoe_block_fwd(a, None, 1, None, 1, nat.BLOCK_NORM, 0.0, 1, 1, 1, 1, None, 1,
                               1 << 20, None) == 1
    assert "NSMOE_BLOCK_NORM" in lib.nsmoe_last_error().decode()
    assert lib.nsmoe_block_fwd(a, norm, None, None, 1, nat.BLOCK_NORM, 0.0, 1, 1, 1, 1, None,
                               1, 1 << 20, None) == 1
    assert "fused router" in lib.nsmoe_last_error().decode()
    #      args norm logits flags coef saved idx counts g g_aux grads w_r gw_r glog ws
    #      ws_bytes stream
    gr = nat.ExpertsGrads(dx=1, dw_in=1, dw_out=1)
    no_grad_w = nat.BlockNorm(weight=1, grad_weight=None, eps=1e-6)
    assert lib.nsmoe_block_bwd(a, no_grad_w, 1, nat.BLOCK_NORM, 0.0, 1, 1, 1, 1, None, gr, 1,
                               1, None, 1, 1 << 20, None) == 1
    assert "grad_weight" in lib.nsmoe_last_error().decode()
