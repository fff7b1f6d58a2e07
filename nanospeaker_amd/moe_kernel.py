"""
HIP (gfx950) dispatch for MoEBlock's dropless path: the drop-in for the reference's
Triton module src/model/moe_kernel.py.

Same public surface as the reference module -- `ALIGN_M`, `KERNEL_ACTIVATIONS`,
`KERNEL_DTYPES`, `kernel_supported`, `fused_moe_forward`, and the custom ops
`moe_dispatch`, `moe_experts` (with its autograd) and `moe_experts_bwd` with the
reference's schemas (moe_kernel.py:180-218, 558-780, 785-803) -- plus the ops this build
adds around them:

  * `route` / `route_bwd`: the softmax / top-k / renormalise tail of TopKRouter.forward
    (src/model/router.py:79-98) and its backward, with CPU torch.topk's tie order;
  * `moe_block` / `moe_block_bwd`: routed *and* shared experts (MoEBlock._shared,
    src/model/moe.py:310-329) in one grouped launch.

Every op enqueues on torch's current stream through the C ABI in include/nsmoe.h
(`_native`); buffers come from torch's caching allocator; nothing syncs with the host.
There is no fallback: on a GPU tensor a missing library raises.
"""

from __future__ import annotations

import ctypes
import threading
import weakref
from collections import OrderedDict
from contextlib import contextmanager, nullcontext
from typing import Optional

import torch
from torch import Tensor

from . import _native as nat

# Each expert's run of dispatch slots is padded to a multiple of ALIGN_M.  The grouped
# GEMMs schedule 64-row tiles per expert on device, so the alignment only has to keep
# the padding small (decode-sized batches would waste most of a 128-row alignment).
ALIGN_M = 16

# Gate activations the kernels implement (ids as in the reference, moe_kernel.py:75).
KERNEL_ACTIVATIONS = {"silu": 0, "swish": 0, "gelu": 1, "relu": 2, "sigmoid": 3, "tanh": 4}

# MFMA input types on gfx950 (bf16 / fp16 16x16x32, fp32 16x16x4); fp64 stays eager.
KERNEL_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# Shape limits of the HIP kernels (include/nsmoe.h).
ROUTE_MAX_EXPERTS = 128
DISPATCH_MAX_EXPERTS = 1024
MAX_GROUPS = 1024

_DT = {torch.bfloat16: nat.BF16, torch.float16: nat.F16, torch.float32: nat.F32}
_DT_TORCH = {v: k for k, v in _DT.items()}


def kernel_supported(t: Tensor) -> bool:
    """
    Whether the fused path takes tensors like this one (device and dtype).  On a GPU
    tensor of a supported dtype the native library must load: a missing build raises
    instead of quietly handing the block to a slower path (moe_kernel.py:81-90 is the
    reference predicate).
    """
    if not (t.is_cuda and t.dtype in KERNEL_DTYPES):
        return False
    if not torch.compiler.is_compiling():  # traced graphs load it when the op first runs
        nat.lib()
    return True


def shape_supported(n_experts: int, n_shared: int, d_hidden: int, dtype: torch.dtype) -> bool:
    """Whether a block of this shape fits the kernels' limits."""
    max_hidden = 128 if dtype == torch.float32 else 256
    return (n_experts <= DISPATCH_MAX_EXPERTS and n_experts + n_shared <= MAX_GROUPS
            and d_hidden <= max_hidden)


def _l_cap(m: int, n_experts: int) -> int:
    """Host worst case for the padded slot count (reference: moe_kernel.py:100-108)."""
    if m <= 0:
        return 0
    return -(-(m + min(n_experts, m) * (ALIGN_M - 1)) // ALIGN_M) * ALIGN_M


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _p(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _ws(nbytes: int, device) -> Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------------------
# router tail
# ---------------------------------------------------------------------------------------

def _route_flags(want_probs: bool, normalize: bool) -> int:
    return (nat.ROUTE_PROBS if want_probs else 0) | (nat.ROUTE_NORMALIZE if normalize else 0)


@torch.library.custom_op("nsmoe::route", mutates_args=())
def route(logits: Tensor, top_k: int, want_probs: bool, normalize: bool,
          w_dtype: int) -> tuple[Tensor, Tensor, Tensor]:
    """
    fp32 logits [T, E] -> (topk_w [T, k] in the dtype coded by w_dtype, topk_idx [T, k]
    int64, probs [T, E] fp32 -- or an empty tensor when want_probs is False).
    """
    logits = logits.contiguous()
    n, e = logits.shape
    dtype = {v: k for k, v in _DT.items()}[w_dtype]
    w = torch.empty((n, top_k), dtype=dtype, device=logits.device)
    idx = torch.empty((n, top_k), dtype=torch.int64, device=logits.device)
    probs = torch.empty((n, e) if want_probs else (0,), dtype=torch.float32, device=logits.device)
    if n:
        nat.check(nat.lib().nsmoe_route_fwd(
            logits.data_ptr(), n, e, top_k, _route_flags(want_probs, normalize), w_dtype,
            w.data_ptr(), idx.data_ptr(), _p(probs), _stream()), "nsmoe_route_fwd")
    return w, idx, probs


@route.register_fake
def _(logits, top_k, want_probs, normalize, w_dtype):
    n, e = logits.shape
    dtype = {v: k for k, v in _DT.items()}[w_dtype]
    return (logits.new_empty((n, top_k), dtype=dtype),
            logits.new_empty((n, top_k), dtype=torch.int64),
            logits.new_empty((n, e) if want_probs else (0,), dtype=torch.float32))


@torch.library.custom_op("nsmoe::route_bwd", mutates_args=())
def route_bwd(src: Tensor, topk_idx: Tensor, grad_w: Tensor, grad_probs: Optional[Tensor],
              want_probs: bool, normalize: bool) -> Tensor:
    """d(logits) [T, E] fp32; `src` is the forward's probs (train branch) or logits."""
    src = src.contiguous()
    n, e = src.shape
    k = topk_idx.shape[1]
    grad_w = grad_w.contiguous()
    gp = grad_probs.contiguous() if grad_probs is not None else None
    out = torch.empty((n, e), dtype=torch.float32, device=src.device)
    if n:
        nat.check(nat.lib().nsmoe_route_bwd(
            src.data_ptr(), topk_idx.contiguous().data_ptr(), grad_w.data_ptr(),
            _DT[grad_w.dtype], _p(gp), None, None, 0.0, n, e, k,
            _route_flags(want_probs, normalize), out.data_ptr(), _stream()), "nsmoe_route_bwd")
    return out


@route_bwd.register_fake
def _(src, topk_idx, grad_w, grad_probs, want_probs, normalize):
    return torch.empty_like(src, dtype=torch.float32)


def _route_setup(ctx, inputs, output):
    logits, top_k, want_probs, normalize, w_dtype = inputs
    w, idx, probs = output
    ctx.want_probs, ctx.normalize = want_probs, normalize
    ctx.w_dtype = w.dtype
    ctx.mark_non_differentiable(idx)
    ctx.save_for_backward(probs if want_probs else logits, idx)


def _route_backward(ctx, grad_w, grad_idx, grad_probs):
    src, idx = ctx.saved_tensors
    if grad_w is None and grad_probs is None:
        return None, None, None, None, None
    if grad_w is None:
        grad_w = torch.zeros(idx.shape, dtype=ctx.w_dtype, device=idx.device)
    if not ctx.want_probs:
        grad_probs = None
    dl = route_bwd(src, idx, grad_w.to(ctx.w_dtype), grad_probs, ctx.want_probs, ctx.normalize)
    return dl, None, None, None, None


route.register_autograd(_route_backward, setup_context=_route_setup)


def route_dtype_code(dtype: torch.dtype) -> int:
    return _DT[dtype]


# ---------------------------------------------------------------------------------------
# dispatch (reference schema: moe_kernel.py:180-218)
# ---------------------------------------------------------------------------------------

@torch.library.custom_op("nsmoe::moe_dispatch", mutates_args=())
def moe_dispatch(topk_idx: Tensor, n_experts: int) -> tuple[
        Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """
    Stable counting sort of the (token, expert) pairs into ALIGN_M-padded expert runs.

    Returns int32 tensors: sorted pair ids [l_cap] (sentinel M in pad slots),
    aligned-block -> expert map [l_cap / ALIGN_M], run offsets [E + 1], routing counts
    [E], the padded total [1] and the inverse pair -> slot [M].  Inside each run the
    pairs are in increasing pair id -- the order of `topk_idx.flatten().sort(stable=True)`
    (moe.py:220) -- so the permutation is deterministic and bit-exact.
    """
    flat = topk_idx.reshape(-1).contiguous().to(torch.int64)
    m = flat.numel()
    dev, i32 = topk_idx.device, torch.int32
    l_cap = _l_cap(m, n_experts)
    sids = torch.empty(l_cap, dtype=i32, device=dev)
    eids = torch.empty(l_cap // ALIGN_M, dtype=i32, device=dev)
    offs = torch.empty(n_experts + 1, dtype=i32, device=dev)
    counts = torch.empty(n_experts, dtype=i32, device=dev)
    npp = torch.empty(1, dtype=i32, device=dev)
    inv = torch.empty(m, dtype=i32, device=dev)
    lib = nat.lib()
    ws = _ws(lib.nsmoe_dispatch_workspace_size(m, n_experts), dev)
    nat.check(lib.nsmoe_dispatch(
        _p(flat), m, n_experts, _p(sids), _p(eids), offs.data_ptr(), counts.data_ptr(),
        npp.data_ptr(), _p(inv), ws.data_ptr(), ws.numel(), _stream()), "nsmoe_dispatch")
    return sids, eids, offs, counts, npp, inv


@moe_dispatch.register_fake
def _(topk_idx, n_experts):
    l_cap = _l_cap(topk_idx.numel(), n_experts)
    mk = lambda n: topk_idx.new_empty((n,), dtype=torch.int32)
    return (mk(l_cap), mk(l_cap // ALIGN_M), mk(n_experts + 1), mk(n_experts), mk(1),
            mk(topk_idx.numel()))


# ---------------------------------------------------------------------------------------
# experts
# ---------------------------------------------------------------------------------------

def _args(x, w_in, w_out, topk_w, b_in, b_out, w_sh_in, w_sh_out, b_sh_in, b_sh_out,
          sorted_ids, pad_offsets, counts, activation) -> nat.ExpertsArgs:
    n, d = x.shape
    return nat.ExpertsArgs(
        dtype=_DT[x.dtype], activation=KERNEL_ACTIVATIONS[activation], n_tokens=n,
        d_model=d, d_hidden=w_in.shape[2] // 2, n_experts=w_in.shape[0],
        n_shared=0 if w_sh_in is None else w_sh_in.shape[0], top_k=topk_w.shape[-1],
        reserved0=0, l_cap=sorted_ids.numel(),
        x=_p(x), w_in=_p(w_in), w_out=_p(w_out), b_in=_p(b_in), b_out=_p(b_out),
        w_sh_in=_p(w_sh_in), w_sh_out=_p(w_sh_out), b_sh_in=_p(b_sh_in), b_sh_out=_p(b_sh_out),
        topk_w=_p(topk_w), sorted_ids=_p(sorted_ids), pad_offsets=_p(pad_offsets),
        counts=_p(counts))


def _c(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None else t.contiguous()


class _PackEntry:
    """One cached pack: weak references to the key tensors and their states, the two
    buffers, the stream they were packed on, what refresh() needs to pack them again, and
    whether a captured graph reads them (then LRU eviction skips the entry)."""

    __slots__ = ("refs", "states", "p_in", "p_out", "stream", "spec", "pinned")

    def __init__(self, refs, states, p_in, p_out, stream, spec):
        self.refs, self.states, self.p_in, self.p_out = refs, states, p_in, p_out
        self.stream, self.spec, self.pinned = stream, spec, False


class PackCache:
    """
    The expert weights' fragment-order packs (nsmoe_pack_weights), kept while the weights
    do not change, so the pack pass (2 x 34.5 MB of traffic at nanoSpeaker's shape) runs
    once per weight update instead of once per forward: eval and decode calls, the
    checkpoint recompute and gradient-accumulation micro-steps all reuse it.

    An entry belongs to the weight tensors themselves (weak references to the objects the
    op was called with) and is valid while each is alive, still at the same storage
    address and shape, and at the same autograd version.  Every in-place write through
    the tensor or a view of it (an optimizer step, load_state_dict, `copy_`) bumps the
    version, and the next call packs into a fresh buffer; an autograd graph that still
    holds the old pack keeps it.  Writes through `.data` bypass the version counter: call
    `clear()` (or `refresh()`) after them.  At most `capacity` weight sets are kept (least
    recently used out); an entry goes as soon as one of its weights is freed.

    * **Casts.** A caller whose parameters are in another dtype than x (an autocast-style
      fp32 master copy with bf16 activations) hands the op cast temporaries that die with
      the call.  `sources({id(temp): param})` names the parameter each temporary was cast
      from for the calls made inside it; the entry is then keyed on the parameters (and
      the packed dtype), so the next call and the checkpoint's recompute hit.
    * **Streams.** A pack is enqueued on the stream current at the miss.  A hit from
      another stream makes that stream wait for the packing stream and marks the buffers
      as used there (`record_stream`), so neither a half-written pack nor a freed one is
      read.
    * **Graphs.** While the current stream is being captured into a HIP graph the cache
      is bypassed by default and the graph packs on every replay.  With
      `share_with_graphs = True` a capture that finds a valid entry reads its buffers
      directly (no pack in the graph: a decode step's replay then moves only the routed
      rows and the weights once), and the entry is pinned: it is no longer evicted, and
      keeps its buffers, until `clear()`.  Such a graph reads whatever the buffers hold
      at replay: after an in-place weight update, call `refresh()` (it repacks every
      live entry into its own buffers, on the current stream) before replaying.  A
      capture that misses still packs inside the graph and files nothing.
    """

    def __init__(self, capacity: int = 64):
        self.capacity = capacity
        self.hits = 0
        self.misses = 0
        self.share_with_graphs = False
        self._lock = threading.RLock()
        self._entries: "OrderedDict[tuple, _PackEntry]" = OrderedDict()
        self._local = threading.local()

    @staticmethod
    def _state(t: Tensor) -> tuple:
        return (t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype, t._version)

    def _drop(self, key) -> None:
        with self._lock:
            self._entries.pop(key, None)

    def clear(self) -> None:
        with self._lock:
            self._entries.clear()

    def __len__(self) -> int:
        return len(self._entries)

    @contextmanager
    def sources(self, mapping: "dict[int, Tensor]"):
        """Within the block, a weight w handed to lookup() with id(w) in `mapping` is keyed
        on mapping[id(w)], the tensor it was cast from."""
        prev = getattr(self._local, "src", None)
        self._local.src = mapping
        try:
            yield
        finally:
            self._local.src = prev

    def _key_tensor(self, w: Tensor) -> Tensor:
        src = getattr(self._local, "src", None)
        return src.get(id(w), w) if src else w

    def lookup(self, nbytes: "tuple[int, int]", device, *weights, spec=None):
        """
        (packed W_in, packed W_out, pending) for these weights (W_in, W_out, W_sh_in,
        W_sh_out; the shared ones may be None).  pending is None on a hit; otherwise the
        buffers are new and still to be packed, and `store(pending, ...)` files them once
        the pack is enqueued.  `spec` = (dtype, d_model, d_hidden, n_experts, n_shared)
        lets refresh() pack the entry again.
        """
        present = tuple(w for w in weights if w is not None)
        cuda = torch.device(device).type == "cuda"
        capturing = cuda and torch.cuda.is_current_stream_capturing()
        pending = None, ()
        if not capturing or self.share_with_graphs:
            keys = tuple(self._key_tensor(w) for w in present)
            key = (tuple(k.data_ptr() for k in keys) + (len(keys),)
                   + tuple(w.dtype for w in present))
            with self._lock:
                entry = self._entries.get(key)
                if entry is not None:
                    if all(r() is k for r, k in zip(entry.refs, keys)) and all(
                            s == self._state(k) for s, k in zip(entry.states, keys)):
                        self._entries.move_to_end(key)
                        self.hits += 1
                        if capturing:
                            entry.pinned = True
                        elif cuda:
                            cur = torch.cuda.current_stream(device)
                            if entry.stream is not None and cur != entry.stream:
                                cur.wait_stream(entry.stream)
                                entry.p_in.record_stream(cur)
                                entry.p_out.record_stream(cur)
                        return entry.p_in, entry.p_out, None
                    if not entry.pinned:
                        del self._entries[key]
            if not capturing:
                pending = key, keys, spec
        self.misses += 1
        p_in = torch.empty(nbytes[0], dtype=torch.uint8, device=device)
        p_out = torch.empty(nbytes[1], dtype=torch.uint8, device=device)
        return p_in, p_out, pending

    def store(self, pending, p_in: Tensor, p_out: Tensor) -> None:
        key, keys = pending[0], pending[1]
        if not keys:
            return
        spec = pending[2] if len(pending) > 2 else None
        cb = lambda _ref, key=key: self._drop(key)
        stream = torch.cuda.current_stream(p_in.device) if p_in.is_cuda else None
        entry = _PackEntry(tuple(weakref.ref(k, cb) for k in keys),
                           tuple(self._state(k) for k in keys), p_in, p_out, stream, spec)
        with self._lock:
            old = self._entries.get(key)
            if old is not None and old.pinned:
                return  # a graph reads the pinned buffers; refresh() updates them
            self._entries[key] = entry
            self._entries.move_to_end(key)
            over = len(self._entries) - self.capacity
            for k in [k for k, e in self._entries.items() if not e.pinned][:max(over, 0)]:
                del self._entries[k]

    def refresh(self) -> int:
        """Pack every live entry again from its weights' current values, into its own
        buffers, on the current stream, and record the new versions.  For graphs captured
        with `share_with_graphs` after an in-place weight update (they hold the buffers'
        addresses).  Returns the number of entries repacked."""
        n = 0
        with self._lock:
            for entry in list(self._entries.values()):
                keys = [r() for r in entry.refs]
                if any(k is None for k in keys) or entry.spec is None:
                    continue
                dt, d, h, e, s = entry.spec
                ws = [k if k.dtype == dt else k.detach().to(dt) for k in keys]
                ws = [w.contiguous() for w in ws]
                a = nat.ExpertsArgs(dtype=_DT[dt], activation=0, n_tokens=0, d_model=d,
                                    d_hidden=h, n_experts=e, n_shared=s, top_k=1,
                                    reserved0=0, l_cap=0, w_in=ws[0].data_ptr(),
                                    w_out=ws[1].data_ptr(),
                                    w_sh_in=ws[2].data_ptr() if s else None,
                                    w_sh_out=ws[3].data_ptr() if s else None)
                nat.check(nat.lib().nsmoe_pack_weights(a, entry.p_in.data_ptr(),
                                                       entry.p_out.data_ptr(), _stream()),
                          "nsmoe_pack_weights")
                entry.states = tuple(self._state(k) for k in keys)
                entry.stream = torch.cuda.current_stream(entry.p_in.device)
                n += 1
        return n


PACKS = PackCache()

# Whether a block forward that autograd will differentiate keeps the experts'
# pre-activations for its backward (NSMOE_BLOCK_SAVE_ACT: rows x 2H elements more of
# `saved` per call, against recomputing x W_in in the backward).  On by default; False
# reproduces the recomputing backward.
SAVE_ACT = True


def _pack_sizes(args: nat.ExpertsArgs) -> "tuple[int, int]":
    nb_in, nb_out = ctypes.c_size_t(), ctypes.c_size_t()
    nat.check(nat.lib().nsmoe_pack_sizes(args, ctypes.byref(nb_in), ctypes.byref(nb_out)),
              "nsmoe_pack_sizes")
    return nb_in.value, nb_out.value


def _pack(args: nat.ExpertsArgs, device, weights):
    """Weights in MFMA fragment order, from the pack cache or packed now: (W_in, W_out)."""
    spec = (_DT_TORCH[args.dtype], args.d_model, args.d_hidden, args.n_experts, args.n_shared)
    p_in, p_out, pending = PACKS.lookup(_pack_sizes(args), device, *weights, spec=spec)
    if pending is not None:
        nat.check(nat.lib().nsmoe_pack_weights(args, p_in.data_ptr(), p_out.data_ptr(),
                                               _stream()), "nsmoe_pack_weights")
        PACKS.store(pending, p_in, p_out)
    args.w_in_packed, args.w_out_packed = p_in.data_ptr(), p_out.data_ptr()
    return p_in, p_out


def _cast_params(dtype: torch.dtype, *params, contiguous: bool = False):
    """(each param cast to dtype -- itself when it already is, and contiguous if asked --,
    {id(cast): param} for the ones that became new tensors): the pack cache keys those on
    the parameters (PackCache.sources), so a cast temporary's pack is found again on the
    next call."""
    out, srcs = [], {}
    for t in params:
        c = None if t is None else t.to(dtype)
        if c is not None and contiguous:
            c = c.contiguous()
        if c is not None and c is not t:
            srcs[id(c)] = t
        out.append(c)
    return out, srcs


def _sources(srcs):
    """PackCache.sources(srcs) for an eager call that cast parameters, else a no-op (a
    traced call's casts are made at run time by the compiled graph)."""
    if srcs and not torch.compiler.is_compiling():
        return PACKS.sources(srcs)
    return nullcontext()


def _check_activation(activation: str) -> None:
    if activation not in KERNEL_ACTIVATIONS:
        raise ValueError(
            f"activation {activation!r} has no kernel; use one of "
            f"{sorted(set(KERNEL_ACTIVATIONS))} or fall back to the eager path.")


def _experts_forward(x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out,
                     topk_w, sorted_ids, pad_offsets, counts, inv_ids, activation):
    """(out, packed W_in); the packed W_in is what the backward needs again."""
    x, w_in, w_out = x.contiguous(), w_in.contiguous(), w_out.contiguous()
    w_sh_in, w_sh_out = _c(w_sh_in), _c(w_sh_out)
    b_in, b_out, b_sh_in, b_sh_out = _c(b_in), _c(b_out), _c(b_sh_in), _c(b_sh_out)
    topk_w = topk_w.reshape(x.shape[0], -1).contiguous()
    n, d = x.shape
    out = torch.empty((n, d), dtype=x.dtype, device=x.device)
    if n == 0:
        return out, x.new_empty(0, dtype=torch.uint8)
    args = _args(x, w_in, w_out, topk_w, b_in, b_out, w_sh_in, w_sh_out, b_sh_in, b_sh_out,
                 sorted_ids, pad_offsets, counts, activation)
    p_in, p_out = _pack(args, x.device, (w_in, w_out, w_sh_in, w_sh_out))
    lib = nat.lib()
    ws = _ws(lib.nsmoe_experts_fwd_workspace_size(args), x.device)
    nat.check(lib.nsmoe_experts_fwd(args, _p(inv_ids), out.data_ptr(), ws.data_ptr(),
                                    ws.numel(), _stream()), "nsmoe_experts_fwd")
    return out, p_in


def _experts_backward(grad_out, x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in,
                      topk_w, sorted_ids, pad_offsets, counts, inv_ids, activation,
                      need_db_in, need_db_out, need_db_sh_in, need_db_sh_out,
                      w_in_packed: Optional[Tensor] = None):
    grad_out = grad_out.to(x.dtype).contiguous()
    x, w_in, w_out = x.contiguous(), w_in.contiguous(), w_out.contiguous()
    w_sh_in, w_sh_out = _c(w_sh_in), _c(w_sh_out)
    b_in, b_out, b_sh_in = _c(b_in), _c(b_out), _c(b_sh_in)
    tw = topk_w.reshape(x.shape[0], -1).contiguous()
    n, d = x.shape
    e, _, h2 = w_in.shape
    s = 0 if w_sh_in is None else w_sh_in.shape[0]
    dev, dt = x.device, x.dtype
    dx = torch.empty_like(x)
    dw_in, dw_out = torch.empty_like(w_in), torch.empty_like(w_out)
    dw_sh_in = torch.empty_like(w_sh_in) if s else x.new_empty(0)
    dw_sh_out = torch.empty_like(w_sh_out) if s else x.new_empty(0)
    dtw = torch.empty(topk_w.shape, dtype=tw.dtype, device=dev)
    db_in = torch.empty((e, h2), dtype=dt, device=dev) if need_db_in else x.new_empty(0)
    db_out = torch.empty((e, d), dtype=dt, device=dev) if need_db_out else x.new_empty(0)
    db_sh_in = torch.empty((s, h2), dtype=dt, device=dev) if need_db_sh_in else x.new_empty(0)
    db_sh_out = torch.empty((s, d), dtype=dt, device=dev) if need_db_sh_out else x.new_empty(0)
    if n == 0:
        dw_in.zero_(), dw_out.zero_(), dtw.zero_()
        for t in (dw_sh_in, dw_sh_out, db_in, db_out, db_sh_in, db_sh_out):
            t.zero_()
        return dx, dw_in, dw_out, dw_sh_in, dw_sh_out, dtw, db_in, db_out, db_sh_in, db_sh_out
    args = _args(x, w_in, w_out, tw, b_in, b_out, w_sh_in, w_sh_out, b_sh_in, None,
                 sorted_ids, pad_offsets, counts, activation)
    grads = nat.ExpertsGrads(
        dx=_p(dx), dw_in=_p(dw_in), dw_out=_p(dw_out), dw_sh_in=_p(dw_sh_in),
        dw_sh_out=_p(dw_sh_out), dtopk_w=_p(dtw), db_in=_p(db_in), db_out=_p(db_out),
        db_sh_in=_p(db_sh_in), db_sh_out=_p(db_sh_out))
    if w_in_packed is not None and w_in_packed.numel():
        args.w_in_packed = w_in_packed.data_ptr()
    else:
        w_in_packed, _ = _pack(args, dev, (w_in, w_out, w_sh_in, w_sh_out))
    lib = nat.lib()
    ws = _ws(lib.nsmoe_experts_bwd_workspace_size(args), dev)
    nat.check(lib.nsmoe_experts_bwd(args, _p(inv_ids), grad_out.data_ptr(), grads,
                                    ws.data_ptr(), ws.numel(), _stream()), "nsmoe_experts_bwd")
    return dx, dw_in, dw_out, dw_sh_in, dw_sh_out, dtw, db_in, db_out, db_sh_in, db_sh_out


# ---- reference schema: routed experts only (moe_kernel.py:558-780) ----------------------

@torch.library.custom_op("nsmoe::moe_experts", mutates_args=())
def moe_experts(x: Tensor, w_in: Tensor, w_out: Tensor, topk_w: Tensor,
                b_in: Optional[Tensor], b_out: Optional[Tensor], sorted_ids: Tensor,
                expert_ids: Tensor, pad_offsets: Tensor, counts: Tensor, n_post_pad: Tensor,
                inv_ids: Tensor, activation: str) -> Tensor:
    """The routed experts on pre-dispatched pairs: out[t] = sum_j w * expert_j(x[t])."""
    out, _ = _experts_forward(x, w_in, w_out, None, None, b_in, b_out, None, None, topk_w,
                              sorted_ids, pad_offsets, counts, inv_ids, activation)
    return out


@moe_experts.register_fake
def _(x, w_in, w_out, topk_w, b_in, b_out, sorted_ids, expert_ids, pad_offsets, counts,
      n_post_pad, inv_ids, activation):
    return x.new_empty(x.shape)


@torch.library.custom_op("nsmoe::moe_experts_bwd", mutates_args=())
def moe_experts_bwd(grad_out: Tensor, x: Tensor, w_in: Tensor, w_out: Tensor, topk_w: Tensor,
                    b_in: Optional[Tensor], sorted_ids: Tensor, expert_ids: Tensor,
                    pad_offsets: Tensor, counts: Tensor, n_post_pad: Tensor, inv_ids: Tensor,
                    activation: str, need_db_in: bool, need_db_out: bool,
                    b_out: Optional[Tensor] = None
                    ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """
    (dx, dW_in, dW_out, dtopk_w, db_in, db_out); unneeded bias grads come back empty.
    The reference schema plus a trailing optional b_out: dtopk_w then includes the
    <grad_out, b_out> term of d((h W_out + b_out) * w) / dw.
    """
    r = _experts_backward(grad_out, x, w_in, w_out, None, None, b_in, b_out, None, topk_w,
                          sorted_ids, pad_offsets, counts, inv_ids, activation,
                          need_db_in, need_db_out, False, False)
    dx, dw_in, dw_out, _, _, dtw, db_in, db_out, _, _ = r
    return dx, dw_in, dw_out, dtw, db_in, db_out


@moe_experts_bwd.register_fake
def _(grad_out, x, w_in, w_out, topk_w, b_in, sorted_ids, expert_ids, pad_offsets, counts,
      n_post_pad, inv_ids, activation, need_db_in, need_db_out, b_out=None):
    e_n, _, h2 = w_in.shape
    return (torch.empty_like(x), torch.empty_like(w_in), torch.empty_like(w_out),
            torch.empty_like(topk_w),
            x.new_empty((e_n, h2)) if need_db_in else x.new_empty(0),
            x.new_empty((e_n, x.shape[1])) if need_db_out else x.new_empty(0))


def _moe_experts_setup(ctx, inputs, output):
    (x, w_in, w_out, topk_w, b_in, b_out, sorted_ids, expert_ids, pad_offsets,
     counts, n_post_pad, inv_ids, activation) = inputs
    saved = [x, w_in, w_out, topk_w, sorted_ids, expert_ids, pad_offsets, counts,
             n_post_pad, inv_ids]
    saved += [t for t in (b_in, b_out) if t is not None]
    ctx.save_for_backward(*saved)
    ctx.has_b_in, ctx.has_b_out = b_in is not None, b_out is not None
    ctx.activation = activation


def _moe_experts_backward(ctx, grad_out):
    (x, w_in, w_out, topk_w, sorted_ids, expert_ids, pad_offsets, counts,
     n_post_pad, inv_ids, *rest) = ctx.saved_tensors
    it = iter(rest)
    b_in = next(it) if ctx.has_b_in else None
    b_out = next(it) if ctx.has_b_out else None
    dx, dw_in, dw_out, dtw, db_in, db_out = moe_experts_bwd(
        grad_out, x, w_in, w_out, topk_w, b_in, sorted_ids, expert_ids, pad_offsets,
        counts, n_post_pad, inv_ids, ctx.activation, ctx.has_b_in, ctx.has_b_out, b_out)
    return (dx, dw_in, dw_out, dtw, db_in if ctx.has_b_in else None,
            db_out if ctx.has_b_out else None, None, None, None, None, None, None, None)


moe_experts.register_autograd(_moe_experts_backward, setup_context=_moe_experts_setup)


# ---- routed + shared experts in one grouped launch ----------------------------------------

@torch.library.custom_op("nsmoe::moe_block", mutates_args=())
def moe_block(x: Tensor, w_in: Tensor, w_out: Tensor, w_sh_in: Optional[Tensor],
              w_sh_out: Optional[Tensor], b_in: Optional[Tensor], b_out: Optional[Tensor],
              b_sh_in: Optional[Tensor], b_sh_out: Optional[Tensor], topk_w: Tensor,
              sorted_ids: Tensor, pad_offsets: Tensor, counts: Tensor, inv_ids: Tensor,
              activation: str) -> tuple[Tensor, Tensor]:
    """
    Routed plus shared experts: out[t] = sum_j w_tj * expert_j(x[t]) + sum_s shared_s(x[t]).
    Returns (out, W_in packed in fragment order); the second output only carries the
    packed weights to the backward.
    """
    return _experts_forward(x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in,
                            b_sh_out, topk_w, sorted_ids, pad_offsets, counts, inv_ids,
                            activation)


def _packed_in_bytes(x, w_in, w_sh_in) -> int:
    e, d, h2 = w_in.shape
    h = h2 // 2
    hp16 = -(-h // 16) * 16
    hp = 64 if hp16 <= 64 else 128 if hp16 <= 128 else 256
    groups = e + (0 if w_sh_in is None else w_sh_in.shape[0])
    es = 4 if x.dtype == torch.float32 else 2
    return groups * (2 * hp // 16) * (-(-d // 32)) * 64 * 8 * es


@moe_block.register_fake
def _(x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out, topk_w, sorted_ids,
      pad_offsets, counts, inv_ids, activation):
    n = _packed_in_bytes(x, w_in, w_sh_in) if x.shape[0] else 0
    return x.new_empty(x.shape), x.new_empty((n,), dtype=torch.uint8)


@torch.library.custom_op("nsmoe::moe_block_bwd", mutates_args=())
def moe_block_bwd(grad_out: Tensor, x: Tensor, w_in: Tensor, w_out: Tensor,
                  w_sh_in: Optional[Tensor], w_sh_out: Optional[Tensor],
                  b_in: Optional[Tensor], b_out: Optional[Tensor], b_sh_in: Optional[Tensor],
                  topk_w: Tensor, sorted_ids: Tensor, pad_offsets: Tensor, counts: Tensor,
                  inv_ids: Tensor, activation: str, need_db_in: bool, need_db_out: bool,
                  need_db_sh_in: bool, need_db_sh_out: bool,
                  w_in_packed: Optional[Tensor] = None) -> tuple[
                      Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                      Tensor]:
    """(dx, dW_in, dW_out, dW_sh_in, dW_sh_out, dtopk_w, db_in, db_out, db_sh_in, db_sh_out)."""
    return _experts_backward(grad_out, x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in,
                             topk_w, sorted_ids, pad_offsets, counts, inv_ids, activation,
                             need_db_in, need_db_out, need_db_sh_in, need_db_sh_out,
                             w_in_packed)


@moe_block_bwd.register_fake
def _(grad_out, x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, topk_w, sorted_ids,
      pad_offsets, counts, inv_ids, activation, need_db_in, need_db_out, need_db_sh_in,
      need_db_sh_out, w_in_packed=None):
    e, d, h2 = w_in.shape
    s = 0 if w_sh_in is None else w_sh_in.shape[0]
    emp = x.new_empty(0)
    return (torch.empty_like(x), torch.empty_like(w_in), torch.empty_like(w_out),
            torch.empty_like(w_sh_in) if s else emp, torch.empty_like(w_sh_out) if s else emp,
            torch.empty_like(topk_w),
            x.new_empty((e, h2)) if need_db_in else emp,
            x.new_empty((e, d)) if need_db_out else emp,
            x.new_empty((s, h2)) if need_db_sh_in else emp,
            x.new_empty((s, d)) if need_db_sh_out else emp)


def _moe_block_setup(ctx, inputs, output):
    (x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out, topk_w, sorted_ids,
     pad_offsets, counts, inv_ids, activation) = inputs
    out, w_in_packed = output
    ctx.mark_non_differentiable(w_in_packed)
    ctx.has = [t is not None for t in (w_sh_in, b_in, b_out, b_sh_in, b_sh_out)]
    opt = [t for t in (w_sh_in, w_sh_out, b_in, b_out, b_sh_in) if t is not None]
    ctx.save_for_backward(x, w_in, w_out, topk_w, sorted_ids, pad_offsets, counts, inv_ids,
                          w_in_packed, *opt)
    ctx.activation = activation


def _moe_block_backward(ctx, grad_out, grad_packed):
    (x, w_in, w_out, topk_w, sorted_ids, pad_offsets, counts, inv_ids, w_in_packed,
     *opt) = ctx.saved_tensors
    has_sh, has_b_in, has_b_out, has_b_sh_in, has_b_sh_out = ctx.has
    it = iter(opt)
    w_sh_in = next(it) if has_sh else None
    w_sh_out = next(it) if has_sh else None
    b_in = next(it) if has_b_in else None
    b_out = next(it) if has_b_out else None
    b_sh_in = next(it) if has_b_sh_in else None
    (dx, dw_in, dw_out, dw_sh_in, dw_sh_out, dtw, db_in, db_out, db_sh_in,
     db_sh_out) = moe_block_bwd(grad_out, x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out,
                                b_sh_in, topk_w, sorted_ids, pad_offsets, counts, inv_ids,
                                ctx.activation, has_b_in, has_b_out, has_b_sh_in,
                                has_b_sh_out, w_in_packed)
    return (dx, dw_in, dw_out,
            dw_sh_in if has_sh else None, dw_sh_out if has_sh else None,
            db_in if has_b_in else None, db_out if has_b_out else None,
            db_sh_in if has_b_sh_in else None, db_sh_out if has_b_sh_out else None,
            dtw, None, None, None, None, None)


moe_block.register_autograd(_moe_block_backward, setup_context=_moe_block_setup)


# ---------------------------------------------------------------------------------------
# entry points for MoEBlock
# ---------------------------------------------------------------------------------------

def fused_moe_forward(x, w_in, w_out, topk_w, topk_idx, b_in, b_out, activation):
    """
    Dispatch + routed experts; returns (out [N, d_model], counts [n_experts] int32), as
    the reference's entry point (moe_kernel.py:785-803).  Params are cast to x's dtype,
    as autocast would run the eager matmuls.
    """
    _check_activation(activation)
    sids, eids, offs, counts, npp, inv = moe_dispatch(topk_idx, w_in.shape[0])
    (w_in, w_out, b_in, b_out), srcs = _cast_params(x.dtype, w_in, w_out, b_in, b_out)
    with _sources(srcs):
        out = moe_experts(x, w_in, w_out, topk_w.to(x.dtype), b_in, b_out, sids, eids, offs,
                          counts, npp, inv, activation)
    return out, counts


def fused_moe_block_forward(x, w_in, w_out, topk_w, topk_idx, b_in, b_out, w_sh_in,
                            w_sh_out, b_sh_in, b_sh_out, activation):
    """fused_moe_forward with the shared experts folded into the same grouped launch."""
    _check_activation(activation)
    sids, eids, offs, counts, npp, inv = moe_dispatch(topk_idx, w_in.shape[0])
    params, srcs = _cast_params(x.dtype, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in,
                                b_sh_out)
    with _sources(srcs):
        out, _ = moe_block(x, *params, topk_w.to(x.dtype), sids, offs, counts, inv, activation)
    return out, counts


# ---------------------------------------------------------------------------------------
# the whole block as one op per direction (the MoEBlock fast path)
# ---------------------------------------------------------------------------------------

def _al256(b):
    return (b + 255) // 256 * 256


def save_act_supported(dtype: torch.dtype, d: int, h: int) -> bool:
    """Whether the block forward can save the experts' pre-activations for the backward
    (nsmoe.h NSMOE_BLOCK_SAVE_ACT): the shapes where the register-tiled expert kernels
    run -- 16-bit types, d % 64 == 0, h % 16 == 0, h <= 128, and the even step counts
    those kernels unroll by (one pass of 192 output columns per 32-row step of H or 2H)."""
    if dtype not in (torch.bfloat16, torch.float16) or d % 64 or h % 16 or h > 128:
        return False
    npass = -(-d // 192)
    return (npass * -(-h // 32)) % 2 == 0 and (npass * (2 * h // 32)) % 2 == 0 and d >= 128


def block_saved_bytes(n: int, e: int, k: int, dtype: torch.dtype, want_probs: bool,
                      save_act: bool = False, d: int = 0, h: int = 0, s: int = 0,
                      norm: bool = False) -> int:
    """
    Size of the block forward's `saved` buffer (nsmoe_block_saved_layout): gates [n, k],
    probs [n, e] fp32 (train branch), sorted ids [l_cap], block owners [l_cap / 16], run
    offsets [e + 1], the padded total, inv [n k] and -- with save_act, where
    save_act_supported(dtype, d, h) -- the pre-activations, 2 h columns of l_cap rows and
    s times n rows rounded up to 16, and with the norm the normalised input [n, d] and its
    rstd [n] fp32, each part rounded up to 256 bytes.  Written in Python so fake tensors with symbolic n get the
    same size; a CPU test holds it equal to the library's.
    """
    return block_saved_offsets(n, e, k, dtype, want_probs, save_act, d, h, s, norm)[-1]


def block_saved_offsets(n: int, e: int, k: int, dtype: torch.dtype, want_probs: bool,
                        save_act: bool = False, d: int = 0, h: int = 0, s: int = 0,
                        norm: bool = False) -> list:
    """The byte offset of each part of `saved` (nsmoe.h NSMOE_SAVED_*), then the total
    (block_saved_bytes)."""
    es = 4 if dtype == torch.float32 else 2
    m = n * k
    l_cap = _l_cap(m, e)
    act = ((l_cap + s * (-(-n // 16) * 16)) * 2 * h * es
           if save_act and save_act_supported(dtype, d, h) else 0)
    parts = (m * es, n * e * 4 if want_probs else 0, l_cap * 4, (l_cap // ALIGN_M) * 4,
             (e + 1) * 4, 4, m * 4, act, n * d * es if norm else 0, n * 4 if norm else 0)
    offs = [0]
    for b in parts:
        offs.append(offs[-1] + _al256(b))
    return offs


class _BlockPlan:
    """Host state of the block call for one shape: the args struct (dims filled once,
    pointers refilled before every call), the `saved` layout and the workspace sizes."""

    def __init__(self, dt, activation, n, d, h, e, s, k, flags):
        lib = nat.lib()
        self.args = nat.ExpertsArgs(
            dtype=_DT[dt], activation=KERNEL_ACTIVATIONS[activation], n_tokens=n, d_model=d,
            d_hidden=h, n_experts=e, n_shared=s, top_k=k, reserved0=0, l_cap=0)
        self.grads = nat.ExpertsGrads()
        self.norm = nat.BlockNorm()
        offs = (ctypes.c_size_t * nat.BLOCK_NSAVED)()
        total = ctypes.c_size_t()
        nat.check(lib.nsmoe_block_saved_layout(self.args, flags, offs, ctypes.byref(total)),
                  "nsmoe_block_saved_layout")
        self.off = list(offs)
        self.saved_bytes = total.value
        self.fwd_ws = lib.nsmoe_block_fwd_workspace_size(self.args, flags)
        nb_in, nb_out = ctypes.c_size_t(), ctypes.c_size_t()
        nat.check(lib.nsmoe_pack_sizes(self.args, ctypes.byref(nb_in), ctypes.byref(nb_out)),
                  "nsmoe_pack_sizes")
        self.pack_bytes = (nb_in.value, nb_out.value)
        # The router GEMM's backward runs inside nsmoe_block_bwd for 16-bit types when
        # d % 16 == 0 and E % 4 == 0 (E <= 128 always holds here); otherwise in torch.
        self.fuse_router = (dt in (torch.bfloat16, torch.float16) and d % 16 == 0
                            and e % 4 == 0 and e <= 128)
        # The forward's router GEMM runs in the library, fused with the router tail, for
        # 16-bit types with d % 32 == 0, d <= 576, E % 4 == 0, E <= 80 and top_k <= 16.
        self.fuse_route = (self.fuse_router and d % 32 == 0 and d <= 576 and e <= 80
                           and k <= 16)
        self.bwd_ws = lib.nsmoe_block_bwd_workspace_size(self.args, flags,
                                                         int(self.fuse_router))

    def bind(self, x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out):
        a = self.args
        a.x, a.w_in, a.w_out = x.data_ptr(), w_in.data_ptr(), w_out.data_ptr()
        a.w_sh_in, a.w_sh_out = _p(w_sh_in), _p(w_sh_out)
        a.b_in, a.b_out, a.b_sh_in, a.b_sh_out = _p(b_in), _p(b_out), _p(b_sh_in), _p(b_sh_out)
        return a


_PLANS = threading.local()
_PLANS_MAX = 16  # shapes kept per host thread (least recently used out)


def _plan(dt, activation, n, d, h, e, s, k, flags) -> _BlockPlan:
    cache = getattr(_PLANS, "cache", None)
    if cache is None:
        cache = _PLANS.cache = OrderedDict()
    key = (dt, activation, n, d, h, e, s, k, flags)
    plan = cache.get(key)
    if plan is None:
        plan = cache[key] = _BlockPlan(dt, activation, n, d, h, e, s, k, flags)
        while len(cache) > _PLANS_MAX:
            cache.popitem(last=False)
    else:
        cache.move_to_end(key)
    return plan


def _route_bits(dt, want_probs, normalize, save_act=False, norm=False) -> int:
    half = dt in (torch.bfloat16, torch.float16)
    return (_route_flags(want_probs, normalize) | (nat.ROUTE_LOGITS16 if half else 0)
            | (nat.BLOCK_SAVE_ACT if save_act else 0) | (nat.BLOCK_NORM if norm else 0))


def norm_fusable(dtype: torch.dtype, d: int, e: int, k: int) -> bool:
    """Whether the block takes the RMSNorm and residual in its own kernels (nsmoe.h
    NSMOE_BLOCK_NORM): the fused router's shapes -- bf16/fp16, d % 32 == 0, d <= 576,
    E % 4 == 0, E <= 80, top_k <= 16."""
    return (dtype in (torch.bfloat16, torch.float16) and d % 32 == 0 and d <= 576
            and e % 4 == 0 and e <= 80 and k <= 16)


def _block_fwd_impl(x, W_r, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out,
                    top_k, want_probs, normalize, activation, aux_coef, logit_bias=None,
                    save_act=False, norm_w=None, norm_eps=1e-6):
    """
    MoEBlock.forward's kernel path (moe.py:345-418): the router GEMM `x @ W_r` (torch,
    router.py:69), then one C call (nsmoe_block_fwd: router tail, dispatch, routed + shared
    experts with the combine, balance loss).  The weights' fragment-order packs come from
    the pack cache, so the pack pass runs only when the weights changed.

    Returns (out [N, d], aux, counts [E] int32, topk_idx [N, k] int64, logits [N, E],
    saved, packed W_in); the last three only carry state to the backward.  aux is the
    balance loss (fp32) when want_probs, else a zero of x's dtype (router.py:52-54,
    moe.py:367-372).

    `logit_bias` [E] fp32 is a harness hook with no counterpart in the reference router
    (which has no bias): a per-expert offset added to the GEMM's output, the sum rounded
    to the GEMM's dtype, before the router tail.  The skewed-routing workload uses it; its
    gradient is not computed.

    With `save_act` the experts' pre-activations are kept in `saved` for the backward
    (nsmoe.h NSMOE_BLOCK_SAVE_ACT), which then skips recomputing x W_in.

    With `norm_w` [d] (an RMSNorm gain; norm_fusable shapes) x is the residual stream and
    `out` is x + block(rms_norm(x, norm_w, norm_eps)) (nsmoe.h NSMOE_BLOCK_NORM): the
    Block's FFN half, nanospeaker.py:169.
    """
    dev, dt = x.device, x.dtype
    n, d = x.shape
    e, h2 = W_r.shape[1], w_in.shape[2]
    s = 0 if w_sh_in is None else w_sh_in.shape[0]
    flags = _route_bits(dt, want_probs, normalize, save_act, norm_w is not None)
    plan = _plan(dt, activation, n, d, h2 // 2, e, s, top_k, flags)
    if norm_w is not None and not plan.fuse_route:
        raise ValueError("block_fwd: the norm needs the fused router's shapes "
                         "(norm_fusable)")
    bias = None
    if plan.fuse_route:
        logits = torch.empty((n, e), dtype=dt, device=dev)  # written by the router kernel
        if logit_bias is not None:
            bias = logit_bias.to(device=dev, dtype=torch.float32).contiguous()
    else:
        logits = x @ W_r
        if dt not in (torch.bfloat16, torch.float16):
            logits = logits.float()
        if logit_bias is not None:
            logits = (logits.float() + logit_bias.float()).to(logits.dtype)
    saved = torch.empty(plan.saved_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty((n, d), dtype=dt, device=dev)
    counts = torch.empty(e, dtype=torch.int32, device=dev)
    topk_idx = torch.empty((n, top_k), dtype=torch.int64, device=dev)
    # The eval branch's loss is a zero of the dtype, written by the library's dispatch
    # launch into the 4 bytes under it (no fill kernel of its own).
    if want_probs:
        aux_buf = torch.empty((), dtype=torch.float32, device=dev)
        aux = aux_buf
    else:
        aux_buf = torch.empty(4 // dt.itemsize, dtype=dt, device=dev)
        aux = aux_buf[0]
    a = plan.bind(x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out)
    if n:
        p_in, p_out, pending = PACKS.lookup(plan.pack_bytes, dev, w_in, w_out, w_sh_in,
                                            w_sh_out, spec=(dt, d, h2 // 2, e, s))
        a.w_in_packed, a.w_out_packed = p_in.data_ptr(), p_out.data_ptr()
        ws = torch.empty(plan.fwd_ws, dtype=torch.uint8, device=dev)
        nrm = None
        if norm_w is not None:
            nrm = plan.norm
            nrm.weight, nrm.grad_weight, nrm.eps = norm_w.data_ptr(), None, float(norm_eps)
        nat.check(nat.lib().nsmoe_block_fwd(
            a, nrm, W_r.data_ptr() if plan.fuse_route else None, _p(bias), logits.data_ptr(),
            flags | (nat.BLOCK_PACK if pending is not None else 0), aux_coef,
            saved.data_ptr(), topk_idx.data_ptr(), counts.data_ptr(), out.data_ptr(),
            aux_buf.data_ptr(), ws.data_ptr(), plan.fwd_ws, _stream()),
            "nsmoe_block_fwd")
        if pending is not None:
            PACKS.store(pending, p_in, p_out)
    else:
        p_in = torch.empty(plan.pack_bytes[0], dtype=torch.uint8, device=dev)
        counts.zero_()
        aux.zero_()
    return out, aux, counts, topk_idx, logits, saved, p_in


@torch.library.custom_op("nsmoe::block_fwd", mutates_args=())
def block_fwd(x: Tensor, W_r: Tensor, w_in: Tensor, w_out: Tensor, w_sh_in: Optional[Tensor],
              w_sh_out: Optional[Tensor], b_in: Optional[Tensor], b_out: Optional[Tensor],
              b_sh_in: Optional[Tensor], b_sh_out: Optional[Tensor], top_k: int,
              want_probs: bool, normalize: bool, activation: str, aux_coef: float,
              logit_bias: Optional[Tensor] = None, save_act: bool = False,
              norm_w: Optional[Tensor] = None, norm_eps: float = 1e-6
              ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The block's forward as a torch.library op (see _block_fwd_impl)."""
    return _block_fwd_impl(x, W_r, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in,
                           b_sh_out, top_k, want_probs, normalize, activation, aux_coef,
                           logit_bias, save_act, norm_w, norm_eps)


@block_fwd.register_fake
def _(x, W_r, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out, top_k,
      want_probs, normalize, activation, aux_coef, logit_bias=None, save_act=False,
      norm_w=None, norm_eps=1e-6):
    n, d = x.shape
    e = W_r.shape[1]
    s = 0 if w_sh_in is None else w_sh_in.shape[0]
    half = x.dtype in (torch.bfloat16, torch.float16)
    return (x.new_empty((n, d)),
            x.new_empty((), dtype=torch.float32 if want_probs else x.dtype),
            x.new_empty((e,), dtype=torch.int32),
            x.new_empty((n, top_k), dtype=torch.int64),
            x.new_empty((n, e), dtype=x.dtype if half else torch.float32),
            x.new_empty((block_saved_bytes(n, e, top_k, x.dtype, want_probs, save_act, d,
                                           w_in.shape[2] // 2, s, norm_w is not None),),
                        dtype=torch.uint8),
            x.new_empty((_packed_in_bytes(x, w_in, w_sh_in),), dtype=torch.uint8))


def _block_bwd_impl(g_out, g_aux, x, W_r, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in,
                    logits, saved, topk_idx, counts, w_in_packed, top_k, want_probs, normalize,
                    activation, aux_coef, has_b_sh_out, need_dx, need_dW_r, save_act=False,
                    norm_w=None):
    """
    The block's backward in one C call (nsmoe_block_bwd: experts' backward, router tail's
    backward with the balance-loss gradient folded in, and for 16-bit types the router
    GEMM's backward: d(logits) W_r^T fused into the dx combine and x^T d(logits) as a
    split-K kernel; other types finish the router GEMM's backward in torch).

    Returns (dx, dW_r, dW_in, dW_out, dW_sh_in, dW_sh_out, db_in, db_out, db_sh_in,
    db_sh_out, dnorm_w); a gradient with no input (no shared experts, no bias, no norm,
    not needed) comes back as an empty tensor.  With `norm_w`, dx is the residual
    stream's gradient through both the norm and the residual.
    """
    n, d = x.shape
    e, h2 = W_r.shape[1], w_in.shape[2]
    s = 0 if w_sh_in is None else w_sh_in.shape[0]
    dev, dt = x.device, x.dtype
    flags = _route_bits(dt, want_probs, normalize, save_act, norm_w is not None)
    half = bool(flags & nat.ROUTE_LOGITS16)
    plan = _plan(dt, activation, n, d, h2 // 2, e, s, top_k, flags)
    emp = lambda: x.new_empty(0)  # one per absent gradient: outputs may not alias
    g_out = g_out.to(dt).contiguous()
    dx = torch.empty_like(x)
    dw_in, dw_out = torch.empty_like(w_in), torch.empty_like(w_out)
    dw_sh_in = torch.empty_like(w_sh_in) if s else emp()
    dw_sh_out = torch.empty_like(w_sh_out) if s else emp()
    db_in = torch.empty_like(b_in) if b_in is not None else emp()
    db_out = torch.empty_like(b_out) if b_out is not None else emp()
    db_sh_in = torch.empty_like(b_sh_in) if b_sh_in is not None else emp()
    db_sh_out = torch.empty((s, d), dtype=dt, device=dev) if has_b_sh_out else emp()
    dnorm_w = torch.empty_like(norm_w) if norm_w is not None else emp()
    fuse = plan.fuse_router
    dlogits = None if fuse else torch.empty((n, e), dtype=dt if half else torch.float32,
                                            device=dev)
    dW_r = torch.empty_like(W_r) if fuse else None
    if n:
        ga = None
        if want_probs and g_aux is not None:
            ga = g_aux.detach().to(torch.float32).reshape(1).contiguous()
        gr = plan.grads
        gr.dx, gr.dw_in, gr.dw_out = dx.data_ptr(), dw_in.data_ptr(), dw_out.data_ptr()
        gr.dw_sh_in, gr.dw_sh_out, gr.dtopk_w = _p(dw_sh_in), _p(dw_sh_out), None
        gr.db_in, gr.db_out = _p(db_in), _p(db_out)
        gr.db_sh_in, gr.db_sh_out = _p(db_sh_in), _p(db_sh_out)
        ws = torch.empty(plan.bwd_ws, dtype=torch.uint8, device=dev)
        # b_sh_out does not enter the backward (the shared experts have no gate).
        a = plan.bind(x, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, None)
        a.w_in_packed, a.w_out_packed = w_in_packed.data_ptr(), None
        nrm = None
        if norm_w is not None:
            nrm = plan.norm
            nrm.weight, nrm.grad_weight = norm_w.data_ptr(), dnorm_w.data_ptr()
        nat.check(nat.lib().nsmoe_block_bwd(
            a, nrm, logits.data_ptr(), flags, aux_coef, saved.data_ptr(), topk_idx.data_ptr(),
            counts.data_ptr(), g_out.data_ptr(), _p(ga), gr, _p(W_r if fuse else None),
            _p(dW_r), _p(dlogits), ws.data_ptr(), plan.bwd_ws, _stream()), "nsmoe_block_bwd")
    else:
        for t in (dx, dw_in, dw_out, dw_sh_in, dw_sh_out, db_in, db_out, db_sh_in, db_sh_out,
                  dlogits, dW_r, dnorm_w):
            if t is not None:
                t.zero_()
        if norm_w is not None:
            dx.copy_(g_out)  # no tokens: the residual's share only
    if not fuse:
        dl = dlogits if half else dlogits.to(dt)
        dW_r = x.t().mm(dl) if need_dW_r else torch.zeros_like(W_r)
        if need_dx:
            dx.addmm_(dl, W_r.t())
    return (dx, dW_r, dw_in, dw_out, dw_sh_in, dw_sh_out, db_in, db_out, db_sh_in, db_sh_out,
            dnorm_w)


@torch.library.custom_op("nsmoe::block_bwd", mutates_args=())
def block_bwd(g_out: Tensor, g_aux: Optional[Tensor], x: Tensor, W_r: Tensor, w_in: Tensor,
              w_out: Tensor, w_sh_in: Optional[Tensor], w_sh_out: Optional[Tensor],
              b_in: Optional[Tensor], b_out: Optional[Tensor], b_sh_in: Optional[Tensor],
              logits: Tensor, saved: Tensor, topk_idx: Tensor, counts: Tensor,
              w_in_packed: Tensor, top_k: int, want_probs: bool, normalize: bool,
              activation: str, aux_coef: float, has_b_sh_out: bool, need_dx: bool,
              need_dW_r: bool, save_act: bool = False, norm_w: Optional[Tensor] = None
              ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                         Tensor, Tensor]:
    """The block's backward as a torch.library op (see _block_bwd_impl)."""
    return _block_bwd_impl(g_out, g_aux, x, W_r, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out,
                           b_sh_in, logits, saved, topk_idx, counts, w_in_packed, top_k,
                           want_probs, normalize, activation, aux_coef, has_b_sh_out, need_dx,
                           need_dW_r, save_act, norm_w)


@block_bwd.register_fake
def _(g_out, g_aux, x, W_r, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, logits,
      saved, topk_idx, counts, w_in_packed, top_k, want_probs, normalize, activation, aux_coef,
      has_b_sh_out, need_dx, need_dW_r, save_act=False, norm_w=None):
    s = 0 if w_sh_in is None else w_sh_in.shape[0]
    like = lambda t: torch.empty_like(t) if t is not None else x.new_empty(0)
    return (torch.empty_like(x), torch.empty_like(W_r), torch.empty_like(w_in),
            torch.empty_like(w_out), like(w_sh_in), like(w_sh_out), like(b_in), like(b_out),
            like(b_sh_in), x.new_empty((s, x.shape[1])) if has_b_sh_out else x.new_empty(0),
            like(norm_w))


def _block_fwd_setup(ctx, inputs, output):
    (x, W_r, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out, top_k,
     want_probs, normalize, activation, aux_coef, logit_bias, save_act, norm_w,
     norm_eps) = inputs
    out, aux, counts, topk_idx, logits, saved, w_in_packed = output
    ctx.mark_non_differentiable(counts, topk_idx, logits, saved, w_in_packed)
    # Unused output gradients arrive as None instead of materialised zeros.
    ctx.set_materialize_grads(False)
    ctx.has = [t is not None for t in (w_sh_in, b_in, b_out, b_sh_in, norm_w)]
    opt = [t for t in (w_sh_in, w_sh_out, b_in, b_out, b_sh_in, norm_w) if t is not None]
    ctx.save_for_backward(x, W_r, w_in, w_out, logits, saved, topk_idx, counts, w_in_packed,
                          *opt)
    ctx.cfg = (top_k, want_probs, normalize, activation, aux_coef, b_sh_out is not None,
               save_act)


def _block_fwd_backward(ctx, g_out, g_aux, g_counts, g_idx, g_logits, g_saved, g_packed):
    return _block_backward(ctx, g_out, g_aux, block_bwd)


def _block_backward(ctx, g_out, g_aux, bwd):
    x, W_r, w_in, w_out, logits, saved, topk_idx, counts, w_in_packed, *opt = ctx.saved_tensors
    has_sh, has_b_in, has_b_out, has_b_sh_in, has_norm = ctx.has
    it = iter(opt)
    w_sh_in = next(it) if has_sh else None
    w_sh_out = next(it) if has_sh else None
    b_in = next(it) if has_b_in else None
    b_out = next(it) if has_b_out else None
    b_sh_in = next(it) if has_b_sh_in else None
    norm_w = next(it) if has_norm else None
    top_k, want_probs, normalize, activation, aux_coef, has_b_sh_out, save_act = ctx.cfg
    need = ctx.needs_input_grad
    if g_out is None:
        g_out = torch.zeros_like(x)
    (dx, dW_r, dw_in, dw_out, dw_sh_in, dw_sh_out, db_in, db_out, db_sh_in, db_sh_out,
     dnorm_w) = bwd(g_out, g_aux, x, W_r, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out,
                    b_sh_in, logits, saved, topk_idx, counts, w_in_packed, top_k, want_probs,
                    normalize, activation, aux_coef, has_b_sh_out, need[0], need[1], save_act,
                    norm_w)
    opt_grad = lambda present, g: g if present else None
    return (dx if need[0] else None, dW_r if need[1] else None, dw_in, dw_out,
            opt_grad(has_sh, dw_sh_in), opt_grad(has_sh, dw_sh_out),
            opt_grad(has_b_in, db_in), opt_grad(has_b_out, db_out),
            opt_grad(has_b_sh_in, db_sh_in), opt_grad(has_b_sh_out, db_sh_out),
            None, None, None, None, None, None, None, opt_grad(has_norm, dnorm_w), None)


block_fwd.register_autograd(_block_fwd_backward, setup_context=_block_fwd_setup)


class _BlockEager(torch.autograd.Function):
    """The same forward and backward as the nsmoe::block_fwd / block_bwd ops, entered
    without the torch.library dispatch: eager callers take this node (its host cost per
    step is what bounds an eager step at nanoSpeaker's shape), traced callers the ops."""

    @staticmethod
    def forward(ctx, *inputs):
        output = _block_fwd_impl(*inputs)
        _block_fwd_setup(ctx, inputs, output)
        return output

    @staticmethod
    def backward(ctx, g_out, g_aux, g_counts, g_idx, g_logits, g_saved, g_packed):
        return _block_backward(ctx, g_out, g_aux, _block_bwd_impl)


def block_forward(x, router_W, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out,
                  top_k, want_probs, normalize, activation, aux_coef, logit_bias=None,
                  norm_w=None, norm_eps=1e-6):
    """The MoE block on the kernel path: the first five results of block_forward_state."""
    return block_forward_state(x, router_W, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out,
                               b_sh_in, b_sh_out, top_k, want_probs, normalize, activation,
                               aux_coef, logit_bias, norm_w, norm_eps)[:5]


def block_forward_state(x, router_W, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in,
                        b_sh_out, top_k, want_probs, normalize, activation, aux_coef,
                        logit_bias=None, norm_w=None, norm_eps=1e-6):
    """
    The MoE block on the kernel path: (out [N, d], aux_loss, counts [E] int32,
    topk_idx [N, k] int64, logits [N, E]).  aux_loss is the balance loss (fp32) when
    want_probs, else a zero of x's dtype (router.py:52-54, moe.py:367-372); logits are the
    router GEMM's output the routing ran on (not differentiable).  Parameters are cast to
    x's dtype, as the eager matmuls would run.

    With `norm_w` (an RMSNorm gain, eps `norm_eps`) x is the residual stream and `out` is
    x + block(F.rms_norm(x)): in the block's kernels where norm_fusable holds, else as
    those three ops.

    block_forward_state also returns the forward's `saved` buffer and the flags that laid
    it out (block_saved_offsets; None, 0 where the block did not run as one op), so a test
    can read what the backward will read -- the normalised input among it.
    """
    _check_activation(activation)
    if norm_w is not None and not norm_fusable(x.dtype, x.shape[-1], router_W.shape[1],
                                               top_k):
        xn = torch.nn.functional.rms_norm(x, (x.shape[-1],), norm_w.to(x.dtype), norm_eps)
        out, aux, counts, topk_idx, logits, saved, flags = block_forward_state(
            xn, router_W, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out,
            top_k, want_probs, normalize, activation, aux_coef, logit_bias)
        return x + out, aux, counts, topk_idx, logits, saved, flags
    op = block_fwd if torch.compiler.is_compiling() else _BlockEager.apply
    # The pre-activations are saved only for a forward that autograd will run backward
    # through (a checkpointed block's first, gradient-free forward does not save them).
    params = (router_W, w_in, w_out, w_sh_in, w_sh_out, b_in, b_out, b_sh_in, b_sh_out, norm_w)
    save_act = SAVE_ACT and torch.is_grad_enabled() and (
        x.requires_grad or any(t is not None and t.requires_grad for t in params))
    cast, srcs = _cast_params(x.dtype, *params, contiguous=True)
    with _sources(srcs):
        out, aux, counts, topk_idx, logits, saved, _ = op(
            x.contiguous(), *cast[:9], top_k, want_probs, normalize, activation,
            float(aux_coef), logit_bias, save_act, cast[9], float(norm_eps))
    flags = _route_bits(x.dtype, want_probs, normalize, save_act, norm_w is not None)
    return out, aux, counts, topk_idx, logits, saved, flags
