"""BASELINE config 4 as one serving pipeline through the integration's step
protocol (fragpack_amd.integrations.vllm.step, the reference's
backend.py:537-578): 4 prompts x 8192 tokens, 32 query heads over 8 KV heads
(GQA 4), one layer.

Step 1 (prefill): the prompts' K/V are written to staging, the prefill
groups gather each prompt's pages into the BF16 workspace and run the MFMA
prefill kernel, and the 64 completed blocks per prompt are encoded.
Step 2 (decode): one new token per sequence, decode attention over the 64
compressed blocks plus the fresh raw tail.

Checked: prefill rows (64 sampled per prompt, first and last included) and
every decode row against fp32 causal attention over the written KV (2e-2 abs
+ 1e-2 rel); the store lost nothing and encoded 4 x 64 blocks x 16 records;
every completed block gathers back bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import workloads
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

S, P, H, G, T, D = 4, 8192, 8, 4, 128, 128
ATOL, RTOL = 2e-2, 1e-2


def _reference(torch, q, k, v, qpos):
    """fp32 causal attention of queries at positions ``qpos`` over k / v [n, H, D]."""
    kf = k.float().repeat_interleave(G, dim=1)
    vf = v.float().repeat_interleave(G, dim=1)
    s = torch.einsum("qhd,khd->hqk", q.float(), kf) * D ** -0.5
    s = s.masked_fill(torch.arange(k.shape[0], device=q.device)[None, None, :] > qpos[None, :, None], float("-inf"))
    return torch.einsum("hqk,khd->qhd", s.softmax(-1), vf)


def test_config4_prefill_encode_decode_pipeline():
    import torch

    from fragpack_amd.compression.attn_tables import device_tables
    from fragpack_amd.integrations.vllm.step import FragPackRunner, layer_forward
    from fragpack_amd.ops.hbm_kv import page_bytes

    dev = torch.device("cuda")
    rng = np.random.default_rng(141)
    scales = workloads.channel_scales(rng, H, 0.02)
    tables = device_tables(workloads.calibrated_tables(rng, H, scales), dev)
    gen = torch.Generator(device=dev).manual_seed(141)
    width = P // T + 1
    nb = S * width
    caches = [torch.empty((nb, page_bytes(H)), dtype=torch.uint8, device=dev)]
    runner = FragPackRunner(H, tables, dev, max_tokens=S * P, max_reqs=S, max_model_len=P + T, overflow_records=1024)
    blocks = np.arange(nb, dtype=np.int32).reshape(S, width)
    bt = torch.from_numpy(blocks).to(dev)
    kv = workloads.gen_kv(torch, gen, S * (P + 1), H, torch.from_numpy(scales).float().to(dev)).view(2, S, P + 1, H, D)
    scale = D ** -0.5

    # ---- step 1: the four prompts ----
    qsl = np.arange(0, S * P + 1, P, dtype=np.int64)
    seq = np.full(S, P, np.int64)
    pos = np.arange(P)
    slots = np.concatenate([blocks[s][pos // T] * T + pos % T for s in range(S)]).astype(np.int64)
    md = runner.build(caches, qsl, seq, torch.from_numpy(seq.astype(np.int32)).to(dev), bt,
                      torch.from_numpy(slots).to(dev), np.zeros(0, np.int32))
    print("config4 pipeline: prefill groups", len(md.prefills), flush=True)
    q = torch.randn((S * P, H * G, D), generator=gen, device=dev).to(torch.bfloat16)
    k_new = kv[0, :, :P].reshape(S * P, H, D)
    v_new = kv[1, :, :P].reshape(S * P, H, D)
    out = torch.full_like(q, float("nan"))
    layer_forward(md, 0, q, k_new, v_new, out, scale)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    for s in range(S):
        rows = np.unique(np.concatenate(([0, P - 1], rng.choice(P, 62, replace=False))))
        r = torch.from_numpy(rows).to(dev)
        ref = _reference(torch, q[s * P + r], kv[0, s, :P], kv[1, s, :P], r)
        torch.testing.assert_close(out[s * P + r].float(), ref, atol=ATOL, rtol=RTOL)
    print("config4 pipeline: prefill rows match", flush=True)

    # ---- step 2: one decode token per sequence ----
    qsl = np.arange(S + 1, dtype=np.int64)
    seq = np.full(S, P + 1, np.int64)
    slots = (blocks[:, P // T] * T).astype(np.int64)  # row 0 of a new block
    md = runner.build(caches, qsl, seq, torch.from_numpy(seq.astype(np.int32)).to(dev), bt,
                      torch.from_numpy(slots).to(dev), np.zeros(0, np.int32))
    qd = torch.randn((S, H * G, D), generator=gen, device=dev).to(torch.bfloat16)
    outd = torch.full_like(qd, float("nan"))
    layer_forward(md, 0, qd, kv[0, :, P].contiguous(), kv[1, :, P].contiguous(), outd, scale)
    torch.cuda.synchronize()
    for s in range(S):
        ref = _reference(torch, qd[s : s + 1], kv[0, s], kv[1, s], torch.tensor([P], device=dev))
        torch.testing.assert_close(outd[s : s + 1].float(), ref, atol=ATOL, rtol=RTOL)
    print("config4 pipeline: decode rows match", flush=True)

    store = runner.store
    stats = store.stats()  # raises StoreError if anything was dropped
    assert stats.encoded == S * (P // T) * 2 * H
    full = torch.from_numpy(blocks[:, : P // T].reshape(-1).copy()).to(dev)
    wk = torch.empty((full.numel(), T, H, D), dtype=torch.bfloat16, device=dev)
    wv = torch.empty_like(wk)
    store.gather(0, full, wk, wv)
    want = kv[:, :, :P].reshape(2, S * (P // T), T, H, D)
    assert torch.equal(wk.view(torch.int16), want[0].view(torch.int16))
    assert torch.equal(wv.view(torch.int16), want[1].view(torch.int16))
