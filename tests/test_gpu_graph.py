"""
The block's kernel path inside a captured HIP graph: a training step (forward + autograd
backward) and a forward are captured once and replayed several times, with eager work and
host synchronisations between the replays; every replay must equal an eager step bit for
bit (the kernels are deterministic), which also shows the library records no memsets or
host synchronisations that a replay would not repeat.

Capture follows torch's recipe: warm-up on a side stream, then capture.  The step returns
every gradient (input, router, experts) from torch.autograd.grad, so the captured graph
writes them into its own memory on each replay and nothing is accumulated.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

mk = pytest.importorskip("nanospeaker_amd.moe_kernel")
from nanospeaker_amd import MoEBlock  # noqa: E402
from tests.helpers import lib_options  # noqa: E402

DEV = "cuda"


def _block(T, seed=0):
    torch.manual_seed(seed)
    m = MoEBlock(576, 76, d_ff=192, top_k=6, n_shared=2, capacity_factor=None, fused=False)
    m = m.to(torch.bfloat16).to(DEV).train()
    x = torch.randn(T, 576, device=DEV).to(torch.bfloat16)
    g = torch.randn(T, 576, device=DEV).to(torch.bfloat16)
    return m, x, g


@pytest.mark.parametrize("T", [2048, 8192])
def test_training_step_replays_equal_eager(T):
    m, x, g = _block(T)
    params = list(m.parameters())
    xg = x.detach().requires_grad_(True)

    one = torch.ones((), dtype=torch.float32, device=DEV)

    def step():
        out = m(xg)
        grads = torch.autograd.grad([out, m.aux_loss], [xg] + params, [g, one])
        return out, list(grads)

    print(f"[graph] T={T} warm-up", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print(f"[graph] T={T} capture", flush=True)
    with torch.cuda.graph(graph):
        out, grads = step()
    aux = m.aux_loss  # the captured tensors (eager calls below rebind the attributes)
    got = []
    for r in range(3):
        scratch = torch.randn(T, 576, device=DEV).to(torch.bfloat16)
        with torch.no_grad():
            m(scratch)  # eager work between replays, on other buffers
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"[graph] T={T} replay {r}", flush=True)
        got.append([out.clone(), aux.detach().clone()] + [t.clone() for t in grads])
    # the eager step
    ref_out, ref_grads = step()
    ref = [ref_out.detach(), m.aux_loss.detach()] + ref_grads
    for r, vals in enumerate(got):
        for i, (a, b) in enumerate(zip(vals, ref)):
            assert torch.equal(a, b), f"replay {r}: tensor {i}"


def test_forward_replays_equal_eager():
    m, x, _ = _block(4096, seed=1)
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                m(x)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = m(x)
        got = []
        for r in range(3):
            m(torch.randn_like(x))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got.append(out.clone())
        ref = m(x)
        for r, v in enumerate(got):
            assert torch.equal(v, ref), f"replay {r}"


def test_side_stream_matches_single_stream():
    """With the "side_stream" option the library runs the weight packing and the dW stage
    on a second stream (forked and joined with events); by default everything stays on
    the caller's stream.  Both orders must give the same bits, step after step (the pack
    cache is emptied before each step, so every step packs on the side stream)."""
    m, x, g = _block(8192, seed=2)
    params = list(m.parameters())
    one = torch.ones((), dtype=torch.float32, device=DEV)

    def step():
        mk.PACKS.clear()
        xg = x.detach().requires_grad_(True)
        out = m(xg)
        grads = torch.autograd.grad([out, m.aux_loss], [xg] + params, [g, one])
        return [out.detach(), m.aux_loss.detach()] + list(grads)

    with lib_options(side_stream=1):
        two = [step() for _ in range(2)]
    single = step()
    torch.cuda.synchronize()
    for r, vals in enumerate(two):
        for i, (a, b) in enumerate(zip(vals, single)):
            assert torch.equal(a, b), f"step {r}: tensor {i}"


@pytest.mark.parametrize("T", [1024, 8192])
def test_replay_repacks_weights_updated_in_place(T):
    """The pack cache is bypassed while a graph is captured, so the captured forward packs
    the weights on every replay: an in-place update between replays (an optimizer step
    outside the graph) is seen by the next replay -- with the pack in the place launch
    (T = 1024) and in the router's launch (T = 8192)."""
    m, x, _ = _block(T, seed=3)
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                m(x)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = m(x)
        for r in range(3):
            m.W_in.mul_(0.9)
            m.W_sh_out.add_(0.01)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            ref = m(x)
            assert torch.equal(out, ref), f"replay {r} used stale packed weights"


def _decode_oracle(m, x):
    """The oracle's eval forward of block m on x [T, d] (the block's own logits)."""
    from oracle import moe_ref as R
    fields = ("W_in", "W_out", "W_sh_in", "W_sh_out")
    p = R.Params(m.router.W.detach().cpu(), *(getattr(m, f).detach().cpu() for f in fields))
    return R.block(x.cpu(), p, m.top_k, train=False, fp32=True,
                   logits=m._logits.float().cpu())


def test_decode_graph_reads_shared_packs_and_refresh():
    """A decode step (T = 64, eval) captured with PackCache.share_with_graphs reads the
    cached packs instead of packing in the graph.  Replays match the oracle (routing
    bit-exact, output within the bf16 bar); after an in-place weight update they keep
    the frozen packs until PackCache.refresh(), after which a replay matches the oracle
    of the updated weights."""
    from tests.helpers import assert_close_bf16
    m, _, _ = _block(64, seed=4)
    m.eval()
    x = torch.randn(64, 576, device=DEV).to(torch.bfloat16)
    mk.PACKS.clear()
    mk.PACKS.share_with_graphs = True
    try:
        with torch.no_grad():
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):
                    m(x)  # the first call packs and files the pack
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            h0, m0 = mk.PACKS.hits, mk.PACKS.misses
            graph = torch.cuda.CUDAGraph()
            print("[graph] decode capture with shared packs", flush=True)
            with torch.cuda.graph(graph):
                out = m(x)
            assert (mk.PACKS.hits - h0, mk.PACKS.misses - m0) == (1, 0), \
                "the capture did not read the cached packs"
            for r in range(3):
                m(torch.randn_like(x))  # eager work between replays
                torch.cuda.synchronize()
                graph.replay()
                torch.cuda.synchronize()
                if r == 0:
                    first = out.clone()
                assert torch.equal(out, first), f"replay {r}"
            eager = m(x)
            assert torch.equal(first, eager)
            ref = _decode_oracle(m, x)
            assert torch.equal(m._routing.cpu(), ref.topk_idx), "routing differs"
            assert_close_bf16("decode replay", first.float().cpu(), ref.out)
            # an in-place update: the replay keeps the frozen packs ...
            m.W_in.mul_(0.5)
            m.W_sh_out.add_(0.02)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            stale = out.clone()
            # ... until refresh() repacks into the same buffers
            assert mk.PACKS.refresh() >= 1
            graph.replay()
            torch.cuda.synchronize()
            fresh = out.clone()
            eager2 = m(x)
            assert torch.equal(fresh, eager2), "refreshed replay != eager"
            assert not torch.equal(stale, fresh)
            ref2 = _decode_oracle(m, x)
            assert torch.equal(m._routing.cpu(), ref2.topk_idx), "routing differs"
            assert_close_bf16("decode replay after refresh", fresh.float().cpu(), ref2.out)
    finally:
        mk.PACKS.share_with_graphs = False
        mk.PACKS.clear()
