"""The fused single-token kernel's failure handling and hand-off hygiene.

A fused launch needs every workgroup resident; its waits for other
workgroups are bounded by wall-clock time, and a launch whose wait expired
must end normally with poisoned outputs and a raised error word, never with a
silently wrong result. These tests force that path from the host: with
UQM_OPT_FUSED_WAIT_US = 0 every wait gives up at its first check, so every
workgroup takes the expired path and every kernel still exits normally.

  * a block launch: NaN output rows, routes -1 and weights NaN, the workspace
    status reports the error once and is then clean, and the next launch at
    the normal budget is bit-identical to one on a fresh workspace;
  * a routed-only launch (routes given) and the no-allocation entry point;
  * an expired marker is removed by the next normal launch (so a later launch
    that reaches the same 16-bit epoch cannot inherit it), while the error
    word stays until the status call;
  * hand-off words another layout left behind: words tagged with the next
    launch's epoch, planted after a call of another shape on the same
    workspace, do not reach the next fused launch (it zeroes its hand-off
    region when the layout changed), and the result is bit-identical to a
    fresh workspace (the test checks that its offsets are the ones the
    kernel writes).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from test_gpu_kernels import DEV, note
from uma_qmoe_amd import _native
from uma_qmoe_amd import synthetic as syn

pytestmark = pytest.mark.gpu

SYNC_ERROR, SYNC_EXPIRED, SYNC_EPOCH_BASE, MAX_FUSED_BLOCKS = 4, 5, 64, 1024


@pytest.fixture()
def ext(hip_ext):
    yield hip_ext
    hip_ext.set_option(_native.UQM_OPT_FUSED_WAIT_US, _native.FUSED_WAIT_US_DEFAULT)
    hip_ext.set_option(_native.UQM_OPT_FUSED_DECODE, 1)


def _c2():
    shape = syn.C2
    layer = syn.build_experts(shape, device=DEV, seed=21)
    dense = syn.build_dense(shape, device=DEV, seed=21)
    x = syn.hidden_states(shape, 1, device=DEV, seed=21)
    return shape, layer, dense, x


def _ws(ext, shape, tokens=1, shared=True):
    return ext.new_workspace(DEV, tokens, shape.hidden, shape.intermediate,
                             shape.shared_intermediate if shared else 0, shape.num_experts, shape.top_k)


def _block(ext, shape, layer, dense, x, ws):
    res = ext.moe_layer(layer, dense, x, shape.top_k, shape.norm_topk_prob, workspace=ws)
    torch.cuda.synchronize()
    return [v.cpu().clone() for v in res]


def _words(ws) -> np.ndarray:
    torch.cuda.synchronize()
    return ws[: 4 * (SYNC_EPOCH_BASE + MAX_FUSED_BLOCKS)].cpu().numpy().view(np.uint32)


def _bits_equal(a, b, what):
    for i, (u, v) in enumerate(zip(a, b)):
        assert u.dtype == v.dtype and torch.equal(u.view(torch.int16) if u.dtype == torch.bfloat16 else u,
                                                  v.view(torch.int16) if v.dtype == torch.bfloat16 else v), \
            f"{what}: output {i} differs"


def test_forced_expiry_poisons_the_block_and_reports_once(ext):
    note("poison: forced expiry, c2 block T=1")
    shape, layer, dense, x = _c2()
    reference = _block(ext, shape, layer, dense, x, _ws(ext, shape))
    ws = _ws(ext, shape)
    ext.set_option(_native.UQM_OPT_FUSED_WAIT_US, 0)
    out, logits, weights, indices = _block(ext, shape, layer, dense, x, ws)
    assert bool(torch.isnan(out.float()).all()), "every output row is poisoned"
    assert bool((indices == -1).all()), "routes are -1 when the routing poll expired"
    assert bool(torch.isnan(weights.float()).all()), "weights are NaN when the routing poll expired"
    words = _words(ws)
    assert words[SYNC_ERROR] != 0 and words[SYNC_EXPIRED] != 0
    with pytest.raises(_native.NativeError, match="wait bound"):
        ext.workspace_status(ws)
    words = _words(ws)
    assert words[SYNC_ERROR] == 0 and words[SYNC_EXPIRED] == 0, "the status call clears both words"
    ext.workspace_status(ws)  # clean now
    ext.set_option(_native.UQM_OPT_FUSED_WAIT_US, _native.FUSED_WAIT_US_DEFAULT)
    again = _block(ext, shape, layer, dense, x, ws)
    _bits_equal(again, reference, "normal launch after a poisoned one")
    ext.workspace_status(ws)


def test_expired_marker_is_removed_by_the_next_launch(ext):
    note("poison: expired marker cleared by the next launch")
    shape, layer, dense, x = _c2()
    ws = _ws(ext, shape)
    ext.set_option(_native.UQM_OPT_FUSED_WAIT_US, 0)
    _block(ext, shape, layer, dense, x, ws)
    poisoned_epoch = int(_words(ws)[SYNC_EXPIRED])
    assert poisoned_epoch == int(_words(ws)[SYNC_EPOCH_BASE]), "the marker names the expired launch"
    ext.set_option(_native.UQM_OPT_FUSED_WAIT_US, _native.FUSED_WAIT_US_DEFAULT)
    out = _block(ext, shape, layer, dense, x, ws)[0]
    assert not bool(torch.isnan(out.float()).any())
    words = _words(ws)
    assert words[SYNC_EXPIRED] == 0, "an expired marker of an earlier launch is removed"
    assert words[SYNC_ERROR] != 0, "the error word stays until the status call"
    with pytest.raises(_native.NativeError, match="wait bound"):
        ext.workspace_status(ws)
    ext.workspace_status(ws)


def test_forced_expiry_routed_only_and_noalloc(ext):
    note("poison: routed-only T=1 and noalloc")
    shape, layer, dense, x = _c2()
    gen = torch.Generator().manual_seed(5)
    idx = torch.randperm(shape.num_experts, generator=gen)[: shape.top_k].view(1, -1).to(DEV)
    w = torch.rand(1, shape.top_k, generator=gen).to(torch.bfloat16).to(DEV)
    ws = _ws(ext, shape, shared=False)
    ref = ext.moe_forward(layer, x, idx, w, workspace=_ws(ext, shape, shared=False)).cpu()
    ext.set_option(_native.UQM_OPT_FUSED_WAIT_US, 0)
    got = ext.moe_forward(layer, x, idx, w, workspace=ws).cpu()
    assert bool(torch.isnan(got.float()).all())
    with pytest.raises(_native.NativeError, match="wait bound"):
        ext.workspace_status(ws)
    ext.set_option(_native.UQM_OPT_FUSED_WAIT_US, _native.FUSED_WAIT_US_DEFAULT)
    assert torch.equal(ext.moe_forward(layer, x, idx, w, workspace=ws).cpu().view(torch.int16), ref.view(torch.int16))

    reference = _block(ext, shape, layer, dense, x, _ws(ext, shape))
    ext.noalloc_status()  # whatever earlier tests left is reported and cleared here
    ext.set_option(_native.UQM_OPT_FUSED_WAIT_US, 0)
    out = [v.cpu().clone() for v in ext.moe_layer_noalloc(layer, dense, x, shape.top_k)]
    assert bool(torch.isnan(out[0].float()).all()) and bool((out[3] == -1).all())
    with pytest.raises(_native.NativeError, match="wait bound"):
        ext.noalloc_status()
    ext.noalloc_status()
    ext.set_option(_native.UQM_OPT_FUSED_WAIT_US, _native.FUSED_WAIT_US_DEFAULT)
    again = [v.cpu().clone() for v in ext.moe_layer_noalloc(layer, dense, x, shape.top_k)]
    _bits_equal(again, reference, "noalloc after a poisoned launch")
    ext.noalloc_status()


def _align256(n: int) -> int:
    return (n + 255) // 256 * 256


def _plant_next_epoch(ws, shape) -> None:
    """Fills the c2 fused hand-off region (shared and routed SiLU products,
    router logits) with words that carry the next launch's epoch: bf16 1.0 in
    the product words, logit 1.0 in the logit words. The offsets follow the
    workspace layout: sync words, then [Is] and [k, I] 32-bit product words,
    then [E + 1] 64-bit logit words, each region 256-byte aligned."""
    words = _words(ws)
    last = int(words[SYNC_EPOCH_BASE])
    nxt = (last + 1) & 0xFFFF or 1
    hs = _align256(4 * (SYNC_EPOCH_BASE + MAX_FUSED_BLOCKS))
    hr = hs + _align256(4 * shape.shared_intermediate)
    lgt = hr + _align256(4 * shape.top_k * shape.intermediate)
    n_prod = (lgt - hs) // 4
    prod = torch.full((n_prod,), (nxt << 16) | 0x3F80, dtype=torch.int64).to(torch.int32)
    ws[hs:lgt].copy_(prod.view(torch.uint8).to(DEV))
    logit = np.full(shape.num_experts + 1, (np.uint64(nxt) << np.uint64(32)) | np.uint64(0x3F800000), dtype=np.uint64)
    ws[lgt: lgt + 8 * (shape.num_experts + 1)].copy_(torch.from_numpy(logit.view(np.uint8)).to(DEV))
    torch.cuda.synchronize()


def test_handoff_words_of_another_layout_are_cleared(ext):
    note("hand-off region cleared on a layout change")
    shape, layer, dense, x = _c2()
    reference = _block(ext, shape, layer, dense, x, _ws(ext, shape))
    ws = _ws(ext, shape, tokens=32)
    first = _block(ext, shape, layer, dense, x, ws)
    _bits_equal(first, reference, "first launch")
    # a call of another layout on the same workspace (routed only, 32 tokens)
    gen = torch.Generator().manual_seed(8)
    idx = torch.stack([torch.randperm(shape.num_experts, generator=gen)[: shape.top_k] for _ in range(32)]).to(DEV)
    wts = torch.rand(32, shape.top_k, generator=gen).to(torch.bfloat16).to(DEV)
    xs = syn.hidden_states(shape, 32, device=DEV, seed=4)
    ext.moe_forward(layer, xs, idx, wts, workspace=ws)
    _plant_next_epoch(ws, shape)
    after = _block(ext, shape, layer, dense, x, ws)
    _bits_equal(after, reference, "fused launch after another layout and planted words")
    ext.workspace_status(ws)
    # the planting hit the hand-off words: after a launch, every word of the
    # three regions carries that launch's epoch at the offsets planted above
    _check_region_tags(ws, shape)


def _check_region_tags(ws, shape) -> None:
    torch.cuda.synchronize()
    epoch = int(_words(ws)[SYNC_EPOCH_BASE])
    hs = _align256(4 * (SYNC_EPOCH_BASE + MAX_FUSED_BLOCKS))
    hr = hs + _align256(4 * shape.shared_intermediate)
    lgt = hr + _align256(4 * shape.top_k * shape.intermediate)
    raw = ws[: lgt + 8 * (shape.num_experts + 1)].cpu().numpy()
    shared = raw[hs: hs + 4 * shape.shared_intermediate].view(np.uint32) >> 16
    routed = raw[hr: hr + 4 * shape.top_k * shape.intermediate].view(np.uint32) >> 16
    logits = raw[lgt: lgt + 8 * (shape.num_experts + 1)].view(np.uint64) >> np.uint64(32)
    assert (shared == epoch).all() and (routed == epoch).all() and (logits == epoch).all()
