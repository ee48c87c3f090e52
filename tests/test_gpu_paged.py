"""The plain BF16 paged decode kernel (the baseline arm, fp_paged_decode)
against fp32 softmax attention: GQA 1/2/4/8, ragged lengths including 0, 1,
127, 128, 129, pages in shuffled order, NaN in every cache row past a
sequence's length (must never be read into the result), one split, the
auto split count and the most splits, and repeated calls (the merge
counters must come back to zero)."""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

T, D = 128, 128


def _case(seed, lens, heads, group):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    rng = np.random.default_rng(seed)
    B = len(lens)
    pages = max(1, max(-(-n // T) for n in lens))
    nb = B * pages + 3
    kc = torch.randn((nb, T, heads, D), generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn((nb, T, heads, D), generator=g, device="cuda").to(torch.bfloat16)
    bt = torch.from_numpy(rng.permutation(nb)[: B * pages].reshape(B, pages).astype(np.int32)).cuda()
    for b, n in enumerate(lens):  # poison every row past the length
        for p in range(pages):
            lo = max(0, n - p * T)
            if lo < T:
                kc[bt[b, p], lo:] = float("nan")
                vc[bt[b, p], lo:] = float("nan")
    q = torch.randn((B, heads * group, D), generator=g, device="cuda").to(torch.bfloat16)
    return q, kc, vc, bt, torch.tensor(lens, dtype=torch.int32, device="cuda")


def _reference(q, kc, vc, bt, lens, heads, group):
    import torch

    out = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    for b, n in enumerate(lens.tolist()):
        if n == 0:
            continue
        k = kc[bt[b].long()].reshape(-1, heads, D)[:n].float()
        v = vc[bt[b].long()].reshape(-1, heads, D)[:n].float()
        qb = q[b].float().view(heads, group, D)
        s = torch.einsum("hgd,thd->hgt", qb, k) * D ** -0.5
        out[b] = torch.einsum("hgt,thd->hgd", s.softmax(-1), v).reshape(heads * group, D)
    return out


@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_paged_decode_vs_fp32(group):
    import torch

    from fragpack_amd.ops.paged_attn import paged_decode_attention, paged_splits, paged_workspace

    lens = [0, 1, 127, 128, 129, 1000, 2047, 300]
    heads = 2
    q, kc, vc, bt, lt = _case(40 + group, lens, heads, group)
    ref = _reference(q, kc, vc, bt, lt, heads, group)
    maxlen = max(lens)
    B = len(lens)
    for splits in (1, paged_splits(B, heads, maxlen), -(-maxlen // T)):
        print("paged case", group, splits, flush=True)
        ws = paged_workspace(B, heads, splits, q.device)
        for _ in range(2):
            out = torch.full_like(q, float("nan"))
            paged_decode_attention(q, kc, vc, bt, lt, maxlen, D ** -0.5, out, ws, splits)
            torch.cuda.synchronize()
            torch.testing.assert_close(out.float(), ref, atol=2e-2, rtol=1e-2)
        assert not ws[2].any(), "merge counters must return to zero"


def test_paged_decode_long_context_config1_shape():
    import torch

    from fragpack_amd.ops.paged_attn import paged_decode_attention, paged_splits, paged_workspace

    lens = [8192] * 4
    q, kc, vc, bt, lt = _case(7, lens, 4, 8)
    splits = paged_splits(4, 4, 8192)
    ws = paged_workspace(4, 4, splits, q.device)
    out = torch.empty_like(q)
    paged_decode_attention(q, kc, vc, bt, lt, 8192, D ** -0.5, out, ws, splits)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.float(), _reference(q, kc, vc, bt, lt, 4, 8), atol=2e-2, rtol=1e-2)


def test_paged_decode_skips_pages_outside_the_cache():
    """Device data the host cannot see: a block id outside [0, num_blocks)
    (here -1 and num_blocks + 5) is skipped like a masked page, and a length
    beyond the block table's width is cut to the table -- nothing outside
    the caches or the table row is read."""
    import torch

    from fragpack_amd.ops.paged_attn import paged_decode_attention, paged_workspace

    heads, group = 2, 4
    lens = [512, 512, 512]
    q, kc, vc, bt, lt = _case(77, lens, heads, group)
    nb = kc.shape[0]
    bt_bad = bt.clone()
    bt_bad[0, 1] = -1
    bt_bad[1, 3] = nb + 5
    lt_long = lt.clone()
    lt_long[2] = 4000  # the table has 4 pages: 512 keys are read
    # references: sequence 0 without page 1, sequence 1 without page 3
    keep = [[0, 2, 3], [0, 1, 2], [0, 1, 2, 3]]
    ref = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    for b in range(3):
        k = kc[bt[b, keep[b]].long()].reshape(-1, heads, D).float()
        v = vc[bt[b, keep[b]].long()].reshape(-1, heads, D).float()
        s = torch.einsum("hgd,thd->hgt", q[b].float().view(heads, group, D), k) * D ** -0.5
        ref[b] = torch.einsum("hgt,thd->hgd", s.softmax(-1), v).reshape(heads * group, D)
    for splits in (1, 2, 4):
        print("paged bounds case", splits, flush=True)
        ws = paged_workspace(3, heads, splits, q.device)
        out = torch.full_like(q, float("nan"))
        paged_decode_attention(q, kc, vc, bt_bad, lt_long, 512, D ** -0.5, out, ws, splits)
        torch.cuda.synchronize()
        torch.testing.assert_close(out.float(), ref, atol=2e-2, rtol=1e-2)
