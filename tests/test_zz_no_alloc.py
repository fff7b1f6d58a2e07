"""
nsmoe_dispatch_noalloc, through the C ABI: the dispatch with library-owned scratch gives
the same buffers as nsmoe_dispatch with a caller workspace, bit for bit, on two calls in
a row (the second smaller, so it runs over the first call's leftover scratch), and
rejects sizes past its scratch before launching anything.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

mk = pytest.importorskip("nanospeaker_amd.moe_kernel")
from nanospeaker_amd import _native as nat  # noqa: E402

DEV = "cuda"


def buffers(m, E):
    l_cap = mk._l_cap(m, E)
    i32 = dict(dtype=torch.int32, device=DEV)
    # filled with a marker so an unwritten element would show
    return [torch.full((l_cap,), -7, **i32), torch.full((l_cap // mk.ALIGN_M,), -7, **i32),
            torch.full((E + 1,), -7, **i32), torch.full((E,), -7, **i32),
            torch.full((1,), -7, **i32), torch.full((m,), -7, **i32)]


def run(idx, E, noalloc):
    lib = nat.lib()
    flat = idx.reshape(-1).contiguous()
    m = flat.numel()
    out = buffers(m, E)
    ptrs = [t.data_ptr() if t.numel() else None for t in out]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.nsmoe_dispatch_noalloc(flat.data_ptr(), m, E, *ptrs, stream)
    else:
        ws = torch.empty(max(lib.nsmoe_dispatch_workspace_size(m, E), 1), dtype=torch.uint8,
                         device=DEV)
        rc = lib.nsmoe_dispatch(flat.data_ptr(), m, E, *ptrs, ws.data_ptr(), ws.numel(), stream)
    nat.check(rc, "dispatch_noalloc" if noalloc else "dispatch")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("E,sizes", [(76, (8192, 2048)), (1000, (3000, 700)), (8, (640, 3))])
def test_noalloc_dispatch_matches_workspace_dispatch(E, sizes):
    g = torch.Generator(device="cpu").manual_seed(E)
    for T in sizes:  # the second call is smaller: it reads none of the first call's scratch
        k = min(6, E)
        idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(DEV)
        print(f"[noalloc] E={E} T={T} k={k}", flush=True)
        want = run(idx, E, noalloc=False)
        got = run(idx, E, noalloc=True)
        for name, a, b in zip(("sorted_ids", "expert_ids", "pad_offsets", "counts",
                               "n_post_pad", "inv"), got, want):
            assert torch.equal(a, b), f"{name} differs (E={E}, T={T})"


def test_noalloc_dispatch_rejects_sizes_past_its_scratch():
    lib = nat.lib()
    m = 262145  # 1025 chunks of 256 pairs x 1024 experts x 4 B > 4 MiB
    rc = lib.nsmoe_dispatch_noalloc(1, m, 1024, 1, 1, 1, 1, 1, 1, None)
    assert rc == 1 and "maximum" in lib.nsmoe_last_error().decode()


def test_noalloc_dispatch_of_no_pairs():
    out = run(torch.zeros(0, 2, dtype=torch.int64, device=DEV), 8, noalloc=True)
    assert int(out[4]) == 0 and int(out[3].sum()) == 0 and int(out[2].abs().sum()) == 0


def test_noalloc_dispatch_under_graph_capture():
    """Captured into a HIP graph (after one uncaptured call resolved the scratch address)
    and replayed three times with new routing written into the captured input between
    replays, each replay equals nsmoe_dispatch on that routing."""
    lib = nat.lib()
    E, T, k = 76, 1024, 6
    g = torch.Generator(device="cpu").manual_seed(5)
    draw = lambda: torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(DEV)
    idx = draw()
    run(idx, E, noalloc=True)  # resolves the address outside capture
    flat = idx.reshape(-1).contiguous()
    m = flat.numel()
    out = buffers(m, E)
    ptrs = [t.data_ptr() for t in out]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    print("[noalloc] capture", flush=True)
    with torch.cuda.graph(graph, stream=side):
        rc = lib.nsmoe_dispatch_noalloc(flat.data_ptr(), m, E, *ptrs,
                                        torch.cuda.current_stream().cuda_stream)
    nat.check(rc, "dispatch_noalloc (captured)")
    for rep in range(3):
        new = draw()
        flat.copy_(new.reshape(-1))
        for t in out:
            t.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        want = run(new, E, noalloc=False)
        for name, a, b in zip(("sorted_ids", "expert_ids", "pad_offsets", "counts",
                               "n_post_pad", "inv"), out, want):
            assert torch.equal(a, b), f"{name} differs on replay {rep}"
