"""Causal varlen prefill (HIP MFMA) vs an fp32 torch reference.

The reference backend's prefill is vLLM FlashAttention (backend.py:560-575),
which no reference test pins (its own check is the gather bit-exactness); the
oracle for this floating-point kernel is textbook fp32 softmax attention over
the same paged workspace, causal mask aligned bottom-right.  Tolerance
2e-2 abs + 1e-2 rel (BF16 in / out, BF16 P, fp32 accumulate).  Covers GQA
groups 1/2/4/8, ragged and single-token sequences, chunked prefill (more keys
than queries), non-causal, tails of partial key tiles and pages, and a long
sequence.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

ATOL, RTOL = 2e-2, 1e-2
D, T = 128, 128


def _case(seed, heads, group, q_lens, k_lens):
    import torch

    g = torch.Generator().manual_seed(seed)
    q_lens = np.asarray(q_lens)
    k_lens = np.asarray(k_lens)
    B = q_lens.size
    pages = [(int(n) + T - 1) // T for n in k_lens]
    n_pages = sum(pages) + 3
    perm = torch.randperm(n_pages, generator=g).numpy()
    width = max(1, max(pages))
    bt = np.zeros((B, width), np.int32)
    used = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[used : used + p]
        used += p
    wk = torch.randn(n_pages, T, heads, D, generator=g).to(torch.bfloat16)
    wv = torch.randn(n_pages, T, heads, D, generator=g).to(torch.bfloat16)
    nq = int(q_lens.sum())
    q = torch.randn(nq, heads * group, D, generator=g).to(torch.bfloat16)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return q, wk, wv, bt, cu, k_lens.astype(np.int32)


def _reference(q, wk, wv, bt, cu, k_lens, group, scale, causal):
    import torch

    out = torch.zeros(q.shape, dtype=torch.float32)
    for b in range(k_lens.size):
        q0, q1 = int(cu[b]), int(cu[b + 1])
        kl = int(k_lens[b])
        if q1 == q0:
            continue
        rows = [int(bt[b, j // T]) for j in range(kl)]
        k = wk[rows, [j % T for j in range(kl)]].float()  # [kl, H, D]
        v = wv[rows, [j % T for j in range(kl)]].float()
        qs = q[q0:q1].float()  # [ql, Hq, D]
        ql = q1 - q0
        kh = k.repeat_interleave(group, dim=1)
        vh = v.repeat_interleave(group, dim=1)
        s = torch.einsum("qhd,khd->hqk", qs, kh) * scale
        if causal:
            qi = torch.arange(ql)[:, None]
            kj = torch.arange(kl)[None, :]
            s = s.masked_fill(kj > qi + (kl - ql), float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[q0:q1] = torch.einsum("hqk,khd->qhd", p, vh)
    return out


def _run(seed, heads, group, q_lens, k_lens, causal=True):
    import torch

    from fragpack_amd.ops.prefill_attn import flash_attn_varlen_func

    q, wk, wv, bt, cu, kl = _case(seed, heads, group, q_lens, k_lens)
    scale = D ** -0.5
    dev = torch.device("cuda")
    out = torch.full_like(q, float("nan"), device=dev)
    print("prefill case", seed, heads, group, list(q_lens), list(k_lens), causal, flush=True)
    flash_attn_varlen_func(q=q.to(dev), k=wk.to(dev), v=wv.to(dev), out=out,
                           cu_seqlens_q=torch.from_numpy(cu).to(dev), max_seqlen_q=int(np.max(q_lens)),
                           seqused_k=torch.from_numpy(kl).to(dev), max_seqlen_k=int(np.max(k_lens)),
                           softmax_scale=scale, causal=causal, block_table=torch.from_numpy(bt).to(dev))
    torch.cuda.synchronize()
    ref = _reference(q, wk, wv, bt, cu, kl, group, scale, causal)
    got = out.float().cpu()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got, ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_ragged_groups(group):
    _run(1 + group, heads=2, group=group, q_lens=[1, 37, 128, 300, 64], k_lens=[1, 37, 128, 300, 64])


def test_chunked_prefill_more_keys_than_queries():
    _run(11, heads=2, group=4, q_lens=[5, 100, 129, 1], k_lens=[700, 100, 260, 999])


def test_non_causal():
    _run(12, heads=1, group=8, q_lens=[33, 200], k_lens=[90, 200], causal=False)


def test_long_sequence():
    _run(13, heads=2, group=4, q_lens=[2048], k_lens=[2048])


def test_empty_sequences_in_batch():
    _run(14, heads=2, group=2, q_lens=[0, 17, 0, 130], k_lens=[0, 17, 40, 130])
