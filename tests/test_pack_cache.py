"""
The weight-pack cache's bookkeeping, on CPU tensors (no kernel runs): a pack is reused
only for the same live weight objects at the same version, and is dropped when a weight
is updated in place, reallocated or freed.
"""

import gc

import torch

from nanospeaker_amd.moe_kernel import PackCache


def weights(seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(4, 8, 6, generator=g), torch.randn(4, 3, 8, generator=g), None, None]


def fill(cache, ws):
    p_in, p_out, pending = cache.lookup((16, 8), "cpu", *ws)
    assert pending is not None
    cache.store(pending, p_in, p_out)
    return p_in, p_out


def test_hit_on_the_same_weights():
    cache, ws = PackCache(), weights()
    p_in, p_out = fill(cache, ws)
    q_in, q_out, pending = cache.lookup((16, 8), "cpu", *ws)
    assert pending is None and q_in is p_in and q_out is p_out
    assert cache.hits == 1 and cache.misses == 1


def test_in_place_update_invalidates():
    cache, ws = PackCache(), weights()
    p_in, _ = fill(cache, ws)
    with torch.no_grad():
        ws[1].add_(1.0)                      # an optimizer step bumps the version counter
    q_in, _, pending = cache.lookup((16, 8), "cpu", *ws)
    assert pending is not None and q_in is not p_in
    view = ws[0][0]
    cache.store(pending, q_in, _)
    with torch.no_grad():
        view.mul_(2.0)                       # a write through a view bumps it as well
    assert cache.lookup((16, 8), "cpu", *ws)[2] is not None


def test_other_objects_at_the_same_address_miss():
    cache, ws = PackCache(), weights()
    fill(cache, ws)
    alias = [ws[0].detach(), ws[1], None, None]  # same storage, another tensor object
    assert cache.lookup((16, 8), "cpu", *alias)[2] is not None


def test_freed_weights_drop_their_entry():
    cache, ws = PackCache(), weights()
    fill(cache, ws)
    assert len(cache) == 1
    del ws[0]
    gc.collect()
    assert len(cache) == 0


def test_capacity_evicts_least_recently_used():
    cache = PackCache(capacity=2)
    sets = [weights(i) for i in range(3)]
    for ws in sets:
        fill(cache, ws)
    assert len(cache) == 2
    assert cache.lookup((16, 8), "cpu", *sets[0])[2] is not None   # evicted
    assert cache.lookup((16, 8), "cpu", *sets[2])[2] is None       # kept


def test_shared_weights_are_part_of_the_key():
    cache, ws = PackCache(), weights()
    sh = [torch.randn(2, 8, 6), torch.randn(2, 3, 8)]
    fill(cache, ws[:2] + sh)
    assert cache.lookup((16, 8), "cpu", *ws)[2] is not None
    assert cache.lookup((16, 8), "cpu", *(ws[:2] + sh))[2] is None


def test_cast_temporaries_are_keyed_on_their_parameters():
    """An autocast-style caller hands the op a fresh cast of its fp32 parameters on every
    call; under PackCache.sources the entry belongs to the parameters, so the next
    call's new temporaries hit, and an update of a parameter invalidates it."""
    cache, params = PackCache(), weights()
    present = params[:2]

    def call():
        temps = [t.to(torch.bfloat16) for t in present]
        with cache.sources({id(c): t for c, t in zip(temps, present)}):
            p_in, p_out, pending = cache.lookup((16, 8), "cpu", *temps, None, None)
            if pending is not None:
                cache.store(pending, p_in, p_out)
        return pending is None

    assert not call()           # first call packs
    assert call() and call()    # new temporaries, same parameters: hits
    assert len(cache) == 1
    with torch.no_grad():
        present[0].add_(1.0)
    assert not call()           # the parameter moved on


def test_packed_dtype_is_part_of_the_key():
    cache, params = PackCache(), weights()
    for dt in (torch.bfloat16, torch.float16):
        temps = [t.to(dt) for t in params[:2]]
        with cache.sources({id(c): t for c, t in zip(temps, params)}):
            p_in, p_out, pending = cache.lookup((16, 8), "cpu", *temps)
            assert pending is not None, dt   # a bf16 pack is no fp16 pack
            cache.store(pending, p_in, p_out)
    assert len(cache) == 2


def test_pinned_entries_outlive_eviction():
    """Entries a captured graph reads are pinned: LRU eviction passes over them."""
    cache = PackCache(capacity=1)
    sets = [weights(i) for i in range(3)]
    fill(cache, sets[0])
    next(iter(cache._entries.values())).pinned = True
    fill(cache, sets[1])
    fill(cache, sets[2])
    assert cache.lookup((16, 8), "cpu", *sets[0])[2] is None   # pinned: kept
    assert cache.lookup((16, 8), "cpu", *sets[1])[2] is not None
