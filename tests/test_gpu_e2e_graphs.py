"""The decode path the end-to-end benchmark times, at the benchmark's own shapes.

The engine is built by needle_amd.e2e.build_engine(), as the benchmark builds it: the
random-init Qwen2-0.5B (24 layers, hidden 896, 14/2 heads, head_dim 64, vocab 151936),
decode graphs captured per batch bucket up to 256 rows, max_model_len 1536 (block tables
96 wide), device-resident decode rows.  The engine's own scheduler drives it: 8 of the
benchmark's requests decode at bucket 8, then 40 short prompts join (a mixed prefill +
decode step) and the batch runs at bucket 48, and sequences leave one by one (rows refilled
from the end) while others grow a block at each 16-token edge, down through buckets 32, 24,
... to 1.  The only addition to the captured graphs is a copy of each layer's q/k/v
projections and attention output into tensors the test reads (forward hooks registered on
the model before the engine captures).

Checks, reference needle/model/runner.py:97-161 and needle/backend/engine.py:110-134:
  * every replay: before it, an eager forward of the same padded batch (the rows in the
    device's row order, built on the host from the scheduler's sequences: the same token,
    context length and block table per row, padding rows on the scratch block); the
    replay's logits must match it within |graph - eager| <= 2e-2 + 1e-2 |eager|, so a
    wrong row refill, token, context length or table entry on the device shows;
  * one replay at bucket 8 and one at bucket 48: every layer's attention output against
    the oracle (RoPE as the reference's torch ops, then the decode append and
    _decode_pytorch) from the q/k/v that replay computed, within the attention tolerance,
    and every layer's pool after the replay byte-equal to the oracle's, with no byte
    changed outside the live rows' new slots and the padding rows' scratch block.
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref
from needle_amd import e2e
from needle_amd.backend.request import SamplingParams
from needle_amd.layers.attention import fused_outputs
from needle_amd.model.config import QWEN2_0_5B, ModelConfig
from needle_amd.model.qwen2 import build_model, random_init_

pytestmark = pytest.mark.gpu


class Probe:
    """Hooks that, while a graph is being captured, copy each layer's q/k/v projections (the
    layer's GEMM recomputed on its input) and
    attention output (o_proj's input) into tensors kept here; every replay rewrites them.
    Outside capture they do nothing."""

    def __init__(self, model):
        self.store = {}
        for i, layer in enumerate(model.model.layers):
            att = layer.self_attn
            att.register_forward_pre_hook(self._projections(i, att))
            att.o_proj.register_forward_pre_hook(self._before(i))

    def _projections(self, i, att):
        # the layer's own projection GEMM (fused or not) on its input, run inside the capture
        def hook(_mod, inp):
            if torch.cuda.is_current_stream_capturing():
                x = inp[0]
                outs = fused_outputs(att._qkv, (att.q_proj, att.k_proj, att.v_proj), x)
                for name, out in zip(("q_proj", "k_proj", "v_proj"), outs):
                    self.store[(i, x.shape[0], name)] = out.clone(
                        memory_format=torch.contiguous_format)
        return hook

    def _before(self, i):
        def hook(_mod, inp):
            if torch.cuda.is_current_stream_capturing():
                self.store[(i, inp[0].shape[0], "attn")] = inp[0].clone()
        return hook


def _close(got, want):
    got = got.float().cpu().numpy().astype(np.float64)
    want = want.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    diff = np.abs(got - want)
    return float((diff - (2e-2 + 1e-2 * np.abs(want))).max()), float(diff.max())


class CheckedReplays:
    """Stands in for the runner's captured graphs: each replay() first runs the eager
    forward of the same padded batch, then the graph, then compares (see module doc)."""

    def __init__(self, engine, probe, oracle_buckets):
        self.runner = engine.runner
        self.probe = probe
        self.oracle_buckets = set(oracle_buckets)
        self.replays = {}              # bucket -> count
        self.worst = 0.0
        self.oracle_checked = []       # (bucket, live rows, worst attention |diff|)
        for b, (g, logits) in list(self.runner._graphs.items()):
            self.runner._graphs[b] = (self._replayer(b, g, logits), logits)

    def _replayer(self, bucket, graph, logits):
        outer = self

        class Replay:
            def replay(self):
                outer.replay(bucket, graph, logits)
        return Replay()

    def _eager_padded(self, bucket):
        r = self.runner
        rows = r._rows
        dev = r.device
        seqs = rows.rows
        b = len(seqs)
        ids = [s.last_token for s in seqs] + [0] * (bucket - b)
        ctx = [s.length - 1 for s in seqs] + [0] * (bucket - b)
        table = np.full((bucket, rows.width), rows.scratch, dtype=np.int32)
        for i, s in enumerate(seqs):
            table[i, :len(s.blocks)] = s.blocks
        ctx_t = torch.tensor(ctx, dtype=torch.int32, device=dev)
        cu = torch.arange(bucket + 1, dtype=torch.int32, device=dev)
        return r.model(torch.tensor(ids, dtype=torch.long, device=dev), ctx_t.long(),
                       r.kv_caches, torch.from_numpy(table).to(dev), cu, ctx_t, 1, False)

    def replay(self, bucket, graph, logits):
        rows = self.runner._rows
        b = len(rows.rows)
        assert 0 < b <= bucket
        eager = self._eager_padded(bucket)
        check = bucket in self.oracle_buckets and b > bucket // 2
        if check:
            self.oracle_buckets.discard(bucket)
            torch.cuda.synchronize()
            before = [p.clone() for p in self.runner.kv_caches]
        graph.replay()
        torch.cuda.synchronize()
        excess, diff = _close(logits[:b], eager[:b])
        self.worst = max(self.worst, diff)
        assert excess <= 0, f"bucket {bucket}, {b} rows: graph logits differ by {diff:.4g}"
        self.replays[bucket] = self.replays.get(bucket, 0) + 1
        if check:
            self._against_oracle(bucket, b, before)

    def _against_oracle(self, bucket, b, before):
        r = self.runner
        rows = r._rows
        seqs = list(rows.rows)
        cfg = r.model_config
        h, hkv, d = cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim
        ctx = torch.tensor([s.length - 1 for s in seqs], dtype=torch.int32)
        # the live rows' blocks, renumbered 0..n-1 in a compact host pool
        used = sorted({blk for s in seqs for blk in s.blocks})
        local = {blk: i for i, blk in enumerate(used)}
        width = max(len(s.blocks) for s in seqs)
        table = torch.full((b, width), len(used) - 1, dtype=torch.int32)
        for i, s in enumerate(seqs):
            table[i, :len(s.blocks)] = torch.tensor([local[x] for x in s.blocks])
        ids = torch.tensor(used, dtype=torch.long, device=r.device)
        new_slot = {(s.blocks[(s.length - 1) // 16], (s.length - 1) % 16) for s in seqs}
        allowed = {blk for blk, _ in new_slot} | {rows.scratch}
        cos, sin = r.model.model.rotary_emb.get_cos_sin(ctx.to(r.device).long())
        cos, sin = cos.cpu(), sin.cpu()
        worst = 0.0
        for layer, (pool, old) in enumerate(zip(r.kv_caches, before)):
            st = self.probe.store
            q = st[(layer, bucket, "q_proj")][:b].view(b, h, d).cpu()
            k = st[(layer, bucket, "k_proj")][:b].view(b, hkv, d).cpu()
            v = st[(layer, bucket, "v_proj")][:b].view(b, hkv, d).cpu()
            got = st[(layer, bucket, "attn")][:b].view(b, h, d)
            compact = old.index_select(1, ids).cpu()
            qr, kr = paged_ref.apply_rope(q, k, cos, sin)
            want = paged_ref.decode(qr, kr, v, compact, table, ctx, 1.0 / d ** 0.5, h, hkv, d)
            excess, diff = _close(got, want)
            worst = max(worst, diff)
            assert excess <= 0, f"bucket {bucket}, layer {layer}: attention differs by {diff:.4g}"
            after = pool.index_select(1, ids).cpu()
            assert torch.equal(after.view(torch.int16), compact.view(torch.int16)), \
                f"bucket {bucket}, layer {layer}: pool bytes differ from the oracle's"
            changed = (pool.view(torch.int16) != old.view(torch.int16)).any(dim=(0, 2, 3, 4))
            blocks = set(torch.nonzero(changed).flatten().tolist())
            assert blocks <= allowed, \
                f"bucket {bucket}, layer {layer}: bytes changed in blocks {sorted(blocks - allowed)[:8]}"
        del before
        self.oracle_checked.append((bucket, b, worst))


@torch.no_grad()
def test_benchmark_engine_graph_replays_match_eager_and_the_oracle():
    cfg = ModelConfig(**QWEN2_0_5B)
    model = random_init_(build_model(cfg), e2e.E2E_SEED)
    probe = Probe(model)
    engine = e2e.build_engine(model=model)
    assert engine.runner._rows.width == 96 and max(engine.runner._graphs) == 256
    checked = CheckedReplays(engine, probe, oracle_buckets=(8, 48))

    bench = e2e.requests(8)
    for i, (rid, prompt, _olen) in enumerate(bench):
        engine.add_request(rid, prompt, SamplingParams(temperature=0.0, max_new_tokens=14 + 3 * i))
    rng = np.random.default_rng(21)
    done = {}
    steps = 0
    joined = False
    while engine.has_unfinished_requests():
        if steps == 4 and not joined:
            for j in range(40):
                prompt = rng.integers(0, cfg.vocab_size, int(rng.integers(40, 81))).tolist()
                engine.add_request(f"short-{j}", prompt, SamplingParams(
                    temperature=0.0, max_new_tokens=int(rng.integers(5, 31))))
            joined = True
        done.update(engine.step())
        steps += 1
        assert steps < 200
    assert len(done) == 48
    seen = sorted(checked.replays)
    print(f"benchmark engine: {steps} steps, replays per bucket {checked.replays}, worst "
          f"|graph - eager| {checked.worst:.3g}, oracle checks {checked.oracle_checked}",
          flush=True)
    assert 8 in seen and 48 in seen and len(seen) >= 4
    assert [c[0] for c in checked.oracle_checked] == [8, 48]
