"""
The decoder harness on the GPU (nanospeaker_amd/decoder.py): one pre-norm block with the
HIP MoE block in situ against the same block with the MoE on the reference's eager path
(same weights, same routing), and the blocked window attention against one SDPA call
under the full band mask, at the prefill workload's head shapes.
"""

import copy

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

pytest.importorskip("nanospeaker_amd.moe_kernel")
from nanospeaker_amd.decoder import Decoder, DecoderConfig, band_attention  # noqa: E402

DEV = "cuda"


def test_band_attention_matches_masked_sdpa_on_gpu():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 9, 2048, 64, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(2, 3, 2048, 64, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(2, 3, 2048, 64, generator=g).to(torch.bfloat16).to(DEV)
    pos = torch.arange(2048, device=DEV)
    allowed = (pos[None, :] <= pos[:, None]) & (pos[:, None] - pos[None, :] < 512)
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=allowed,
                                         enable_gqa=True)
    got = band_attention(q, k, v, 512)
    assert_close_bf16("band attention", got.float().cpu(), ref.cpu())


@pytest.mark.parametrize("window", [None, 256])
def test_one_layer_with_hip_moe_matches_the_eager_block(window):
    print(f"[decoder] one layer, window={window}", flush=True)
    torch.manual_seed(0)
    cfg = DecoderConfig(n_layers=1, window=window, global_every=None)
    model = Decoder(cfg).to(torch.bfloat16).to(DEV).eval()
    twin = copy.deepcopy(model)
    for blk in twin.blocks:
        blk.ffn.kernel = False
    idx = torch.randint(0, cfg.vocab_size, (2, 1024), device=DEV)
    with torch.no_grad():
        hk, _ = model.trunk(idx)
        he, _ = twin.trunk(idx)
    assert model.blocks[0].ffn._use_kernel(hk.reshape(-1, 576))
    assert torch.equal(model.blocks[0].ffn.expert_counts.long(),
                       twin.blocks[0].ffn.expert_counts.long())
    # both sides are bf16 computations, each within the bf16 bar (rel-L2 5e-3) of an fp32
    # one, so they are held to twice that against each other
    assert_close_bf16("hidden states", hk.float().cpu(), he.float().cpu(), rel_l2=1e-2)
