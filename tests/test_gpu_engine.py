"""A simulated serving engine driving the store and kernels step by step.

The reference runs its backend only under a real vLLM (its GPU tests drive
HbmKvStore directly).  Here a small engine, written for the test, schedules
requests over a shared block pool as vLLM's V2 runner does: chunked prefill,
decodes first in the batch, blocks allocated per step and freed (LIFO, so a
finished request's partially written block goes straight to a new request),
a preempted request re-admitted with a new allocation and recomputed.  Each
step runs every layer through the integration (write -> decode attention over
compressed records -> workspace gather + prefill -> encode -> commit), and
each layer's output is compared with fp32 causal attention over that layer's
full KV history (2e-2 abs + 1e-2 rel, in units of each V channel's scale).  At the end the store reports no lost
data, its encode counter equals the records of every block closed, and every
full block of a running request decodes bit-exact to the KV written.

Two drivers: ``core`` calls ``step.FragPackRunner`` / ``layer_forward``
directly; ``vllm`` goes through the backend classes (builder, impl, runner
wrapper feeding the open-block tracker) against the stand-in vLLM modules.
"""

from __future__ import annotations

import importlib
import math
from types import SimpleNamespace

import numpy as np
import pytest

from tests import fake_vllm, workloads
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

ATOL, RTOL = 2e-2, 1e-2
T, D = 128, 128
L, H, G = 3, 2, 4
NB = 48
MAX_LEN = 1024  # the core driver keeps an 8-page prefill workspace: two long prefills need two passes
MAX_TOKENS = 2048
MAX_REQS = 8
WIDTH = MAX_LEN // T

# (new requests {id: prompt}, scheduled tokens {id: n}, finished, preempted)
SCHEDULE = [
    ({"a": 254, "b": 766}, {"a": 254, "b": 200}, (), ()),
    ({}, {"a": 1, "b": 566}, (), ()),  # a decodes, b finishes its prompt in a 566-token chunk
    ({"c": 126}, {"a": 1, "b": 1, "c": 126}, (), ()),  # a closes block 1
    ({}, {"a": 1, "b": 1, "c": 1}, (), ()),  # b closes block 5
    ({"d": 600, "e": 900}, {"b": 1, "c": 1, "d": 600, "e": 900}, ("a",), ()),  # a's open block goes to d
    ({}, {"b": 1, "c": 1, "d": 1, "e": 1}, (), ()),
    ({}, {"c": 1, "d": 1, "e": 1}, (), ("b",)),  # b preempted
    ({"b": None}, {"d": 1, "e": 1, "b": None}, ("c",), ()),  # c done; b recomputed from scratch
    ({}, {"b": 1, "d": 1, "e": 1}, (), ()),
]


class Engine:
    def __init__(self, driver: str, monkeypatch, tmp_path):
        import torch

        from fragpack_amd.compression.attn_tables import device_tables
        from fragpack_amd.ops.hbm_kv import page_bytes

        self.torch = torch
        self.dev = torch.device("cuda")
        self.driver = driver
        rng = np.random.default_rng(61)
        self.scales = torch.from_numpy(workloads.channel_scales(rng, H, 0.02)).float()
        tables = np.repeat(workloads.calibrated_tables(rng, H, self.scales.numpy()), L, axis=0)  # [L, 2, H, 22]
        self.gen = torch.Generator().manual_seed(62)
        self.caches = [torch.empty((NB, page_bytes(H)), dtype=torch.uint8, device=self.dev) for _ in range(L)]
        self.names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
        self.scale = D ** -0.5
        self.free = list(range(NB - 1, -1, -1))  # pop() hands out the most recently freed block
        self.blocks: dict[str, list[int]] = {}
        self.computed: dict[str, int] = {}
        self.hist: dict[str, list] = {}  # per request: [L] of [2, len, H, D] bf16 on the GPU
        self.closes = 0
        if driver == "core":
            from fragpack_amd.integrations.vllm.lifecycle import OpenBlocks
            from fragpack_amd.integrations.vllm.step import FragPackRunner

            self.tracker = OpenBlocks(T)
            self.runner = FragPackRunner(H, device_tables(tables, self.dev), self.dev, MAX_TOKENS, MAX_REQS,
                                         MAX_LEN, overflow_records=64, workspace_pages=WIDTH)
        else:
            self.fakes = fake_vllm.install(monkeypatch)
            path = tmp_path / "tables.npz"
            np.savez(path, table=tables)
            monkeypatch.setenv("FRAGPACK_TABLES", str(path))
            monkeypatch.setenv("FRAGPACK_OVERFLOW", "64")
            self.backend = importlib.import_module("fragpack_amd.integrations.vllm.backend")
            cfg = fake_vllm.VllmConfig(
                scheduler_config=SimpleNamespace(max_num_batched_tokens=MAX_TOKENS, max_num_seqs=MAX_REQS),
                model_config=SimpleNamespace(max_model_len=MAX_LEN),
                layers={n: fake_vllm.Attention(n, c) for n, c in zip(self.names, self.caches)},
            )
            spec = fake_vllm.AttentionSpec(block_size=T, num_kv_heads=H, head_size=D)
            self.builder = self.backend.FragPackMetadataBuilder(spec, list(reversed(self.names)), cfg, self.dev)
            self.impl = self.backend.FragPackAttentionImpl(H * G, D, self.scale, H)
            self.model_runner = self.fakes.GPUModelRunner()

    def _kv(self, n):
        x = self.torch.randn((2, n, H, D), generator=self.gen) * self.scales[:, None]
        return x.to(self.torch.bfloat16).to(self.dev)

    def step(self, new, sched, finished, preempted):
        torch = self.torch
        gone = set(finished) | set(preempted)
        for r in gone:
            self.free.extend(self.blocks.pop(r))
            del self.computed[r]
            if r in finished:
                del self.hist[r]
        so_new, so_cached = [], ([], [], [])
        new_blocks = {}
        rows = sorted(sched, key=lambda r: sched[r] != 1)  # decodes first (a recompute is a prefill)
        qlens = []
        for r in rows:
            if r in new:
                self.blocks[r], self.computed[r] = [], 0
                if r not in self.hist:
                    self.hist[r] = [torch.empty((2, 0, H, D), dtype=torch.bfloat16, device=self.dev)] * L
            c = self.computed[r]
            n = sched[r] if sched[r] is not None else self.hist[r][0].shape[1]  # recompute everything
            need = math.ceil((c + n) / T) - len(self.blocks[r])
            got = [self.free.pop() for _ in range(max(need, 0))]
            self.blocks[r].extend(got)
            new_blocks[r] = got
            qlens.append(n)
        for r in rows:
            if r in new:
                so_new.append(SimpleNamespace(req_id=r, block_ids=(list(self.blocks[r]),), num_computed_tokens=0))
            else:
                so_cached[0].append(r)
                so_cached[1].append(self.computed[r])
                so_cached[2].append((new_blocks[r],) if new_blocks[r] else None)
        so = SimpleNamespace(
            finished_req_ids=set(finished), preempted_req_ids=set(preempted), scheduled_new_reqs=so_new,
            block_table_updates=None,
            scheduled_cached_reqs=SimpleNamespace(req_ids=so_cached[0], num_computed_tokens=so_cached[1],
                                                  new_block_ids=so_cached[2], resumed_req_ids=set()))
        qlens = np.array(qlens, np.int64)
        qsl = np.concatenate(([0], np.cumsum(qlens)))
        prior = np.array([self.computed[r] for r in rows], np.int64)
        seq = prior + qlens
        ntok = int(qsl[-1])
        self.closes += int(np.sum(seq // T - prior // T))
        slots = np.full(ntok + 3, -1, np.int64)  # padded like a graph-shaped batch
        bt = np.zeros((len(rows), WIDTH), np.int32)
        for i, r in enumerate(rows):
            pos = np.arange(prior[i], seq[i])
            slots[qsl[i] : qsl[i + 1]] = np.asarray(self.blocks[r])[pos // T] * T + pos % T
            bt[i, : len(self.blocks[r])] = self.blocks[r]
        slot_d = torch.from_numpy(slots).to(self.dev)
        bt_d = torch.from_numpy(bt).to(self.dev)
        seq_d = torch.from_numpy(seq.astype(np.int32)).to(self.dev)
        print("step", rows, qlens.tolist(), seq.tolist(), flush=True)
        if self.driver == "core":
            self.tracker.update(so)
            md = self.runner.build(self.caches, qsl, seq, seq_d, bt_d, slot_d, self.tracker.live_blocks())
        else:
            self.model_runner.execute_model(so)  # the wrapper feeds the backend's tracker
            cam = fake_vllm.CommonAttentionMetadata(
                query_start_loc=torch.from_numpy(qsl.astype(np.int32)).to(self.dev),
                query_start_loc_cpu=torch.from_numpy(qsl.astype(np.int32)),
                seq_lens=seq_d, seq_lens_cpu_upper_bound=torch.from_numpy(seq.astype(np.int32)),
                num_reqs=len(rows), num_actual_tokens=ntok, block_table_tensor=bt_d, slot_mapping=slot_d)
            md = self.builder.build(0, cam)
        recompute = {r for r in rows if sched[r] is None}
        vs = self.scales[1].repeat_interleave(G, dim=0).to(self.dev)  # [H * G, D]
        for li in range(L):
            q = torch.randn((ntok, H * G, D), generator=self.gen).to(torch.bfloat16).to(self.dev)
            kv = torch.empty((2, ntok, H, D), dtype=torch.bfloat16, device=self.dev)
            for i, r in enumerate(rows):
                if r in recompute:
                    kv[:, qsl[i] : qsl[i + 1]] = self.hist[r][li]
                else:
                    kv[:, qsl[i] : qsl[i + 1]] = self._kv(int(qlens[i]))
                    self.hist[r][li] = torch.cat((self.hist[r][li], kv[:, qsl[i] : qsl[i + 1]]), dim=1)
            out = torch.full((ntok, H * G, D), float("nan"), dtype=torch.bfloat16, device=self.dev)
            if self.driver == "core":
                from fragpack_amd.integrations.vllm.step import layer_forward

                layer_forward(md, li, q, kv[0], kv[1], out, self.scale)
            else:
                self.impl.forward(SimpleNamespace(layer_name=self.names[li]), q, kv[0], kv[1], self.caches[li],
                                  md, out)
            torch.cuda.synchronize()
            for i, r in enumerate(rows):
                ref = self._reference(q[qsl[i] : qsl[i + 1]], self.hist[r][li][:, : seq[i]], int(prior[i]))
                got = out[qsl[i] : qsl[i + 1]].float()
                assert torch.isfinite(got).all(), (r, li)
                # in units of each V channel's scale: BF16 rounding of P and of
                # the output scales with |V|, which the channel scales vary
                torch.testing.assert_close(got / vs, ref / vs, atol=ATOL, rtol=RTOL,
                                           msg=lambda m: f"{r} layer {li}: {m}")
        for r in rows:
            self.computed[r] = int(seq[rows.index(r)])

    def _reference(self, q, kv, prior):
        torch = self.torch
        k = kv[0].float().repeat_interleave(G, dim=1)
        v = kv[1].float().repeat_interleave(G, dim=1)
        s = torch.einsum("qhd,khd->hqk", q.float(), k) * self.scale
        qpos = prior + torch.arange(q.shape[0], device=self.dev)
        s = s.masked_fill(torch.arange(k.shape[0], device=self.dev)[None, None, :] > qpos[None, :, None],
                          float("-inf"))
        return torch.einsum("hqk,khd->qhd", s.softmax(-1), v)

    def store(self):
        if self.driver == "core":
            return self.runner.store
        return self.builder.runner.store

    def finish_checks(self):
        torch = self.torch
        store = self.store()
        stats = store.stats()  # raises StoreError on lost data
        print("store", stats, "closes", self.closes, flush=True)
        assert stats.encoded == self.closes * 2 * H * L
        for r, blocks in self.blocks.items():
            full = self.computed[r] // T
            if not full:
                continue
            ids = torch.tensor(blocks[:full], dtype=torch.int32, device=self.dev)
            for li in range(L):
                wk = torch.empty((full, T, H, D), dtype=torch.bfloat16, device=self.dev)
                wv = torch.empty_like(wk)
                store.gather(li, ids, wk, wv)
                want = self.hist[r][li][:, : full * T].reshape(2, full, T, H, D)
                assert torch.equal(wk.view(torch.int16), want[0].view(torch.int16)), (r, li)
                assert torch.equal(wv.view(torch.int16), want[1].view(torch.int16)), (r, li)


@pytest.mark.parametrize("driver", ["core", "vllm"])
def test_engine_steps_match_fp32_attention(driver, monkeypatch, tmp_path):
    eng = Engine(driver, monkeypatch, tmp_path)
    for i, step in enumerate(SCHEDULE):
        print("schedule step", i, flush=True)
        eng.step(*step)
    eng.finish_checks()
    from fragpack_amd.integrations.vllm.capacity import get_capacity

    cap = get_capacity()
    assert cap is not None and cap.blocks == NB and cap.layers == L and cap.kv_heads == H
    assert cap.memory["arena"] == NB * L * cap.page_bytes
