"""Host-side pieces of the continuous-batching driver: sampler, batch metadata and the
bookkeeping of the device-resident decode rows (run against a CPU buffer here)."""
import random

import pytest
import torch

from needle_amd.backend.request import SamplingParams, SeqState
from needle_amd.model.config import ModelConfig
from needle_amd.model.runner import ModelRunner, _DecodeRows
from needle_amd.model.sampler import sample


def test_greedy_sampling_and_refused_stochastic_rows():
    torch.manual_seed(0)
    logits = torch.randn(5, 50)
    want = logits.argmax(-1).tolist()
    assert sample(logits, [SamplingParams(temperature=0.0)] * 5) == want
    for p in (SamplingParams(), SamplingParams(temperature=0.7, top_k=1)):
        with pytest.raises(NotImplementedError):
            sample(logits, [SamplingParams(temperature=0.0)] * 4 + [p])


def test_sampling_params_reject_out_of_range_values():
    for bad in (dict(temperature=-1.0), dict(top_p=0.0), dict(top_p=1.5),
                dict(max_new_tokens=0)):
        try:
            SamplingParams(**bad)
        except ValueError:
            continue
        raise AssertionError(f"accepted {bad}")


def _seq(seq_id, toks, gen=0, blocks=()):
    s = SeqState(seq_id, f"r{seq_id}", list(toks[:len(toks) - gen]),
                 SamplingParams(temperature=0))
    s.tokens = list(toks)
    s.blocks = list(blocks)
    return s


def test_prepare_inputs_follows_the_reference_rules():
    # runner.py:194-249: prefill = every token at context 0; decode = the newest token at
    # context length-1; positions ctx..; cu_seqlens; rows padded with num_blocks - 1
    cfg = ModelConfig(hidden_size=128, num_hidden_layers=1, num_attention_heads=2,
                      num_key_value_heads=1, intermediate_size=64, vocab_size=32,
                      max_position_embeddings=64)
    r = ModelRunner(cfg, device="cpu")
    r.init_kv_cache(10)
    a = _seq(1, list(range(5)), blocks=[3])
    b = _seq(2, list(range(20)), blocks=[7, 2])
    inp = r.prepare_inputs([a, b], is_prefill=True)
    assert inp.input_ids.tolist() == list(range(5)) + list(range(20))
    assert inp.positions.tolist() == list(range(5)) + list(range(20))
    assert inp.cu_seqlens.tolist() == [0, 5, 25] and inp.cu_seqlens.dtype == torch.int32
    assert inp.context_lens.tolist() == [0, 0] and inp.context_lens.dtype == torch.int32
    assert inp.block_table.tolist() == [[3, 9], [7, 2]] and inp.block_table.dtype == torch.int32
    assert inp.max_seqlen == 20 and inp.is_prefill
    inp = r.prepare_inputs([a, b], is_prefill=False)
    assert inp.input_ids.tolist() == [4, 19] and inp.positions.tolist() == [4, 19]
    assert inp.context_lens.tolist() == [4, 19] and inp.cu_seqlens.tolist() == [0, 1, 2]
    assert inp.max_seqlen == 1 and not inp.is_prefill


def _expect(rows: _DecodeRows, seqs, tokens_on_device):
    """The dense layout the device buffer must hold after sync(seqs)."""
    cap, w = rows.capacity, rows.width
    tok = tokens_on_device.clone()
    ctx = torch.zeros(cap, dtype=torch.int32)
    tab = torch.full((cap, w), rows.scratch, dtype=torch.int32)
    where = rows.row_of()
    assert sorted(where.values()) == list(range(len(seqs)))
    for s in seqs:
        r = where[id(s)]
        ctx[r] = s.length - 1
        tab[r, :len(s.blocks)] = torch.tensor(s.blocks, dtype=torch.int32)
        tok[r] = s.last_token
    return tok, ctx, tab


def test_decode_rows_track_joins_leaves_and_growth():
    """A random run of arriving, leaving and growing sequences: after every sync the buffer
    holds exactly the live sequences' rows, and padding rows hold (0, 0, scratch...)."""
    rng = random.Random(4)
    cap, width, scratch = 12, 9, 99
    rows = _DecodeRows(cap, width, scratch, "cpu")
    live, next_id = [], 1
    for step in range(300):
        # leave / arrive
        for s in list(live):
            if rng.random() < 0.08:
                live.remove(s)
        while len(live) < cap and rng.random() < 0.3:
            n = rng.randint(1, 100)
            s = _seq(next_id, [rng.randint(0, 1000) for _ in range(n)],
                     blocks=rng.sample(range(scratch), (n + 15) // 16))
            next_id += 1
            live.append(s)
        rng.shuffle(live)
        if not live:
            continue
        rows.sync(live)
        before_tok = rows.tok.clone()
        tok, ctx, tab = _expect(rows, live, before_tok)
        assert torch.equal(rows.ctx, ctx) and torch.equal(rows.table, tab)
        b = len(live)
        assert torch.equal(rows.tok[:b], tok[:b])
        assert (rows.ctx[b:] == 0).all() and (rows.table[b:] == scratch).all()
        # a "replay": the greedy token of every live row lands on the device and on the host
        for s in live:
            t = rng.randint(0, 1000)
            rows.tok[rows.row_of()[id(s)]] = t
            s.tokens.append(t)
            if (s.length + 15) // 16 > len(s.blocks) and len(s.blocks) < width:
                s.blocks.append(rng.randrange(scratch))
        for r in range(b):
            rows.tok_on_device[r] = True
        # sequences past the table width leave (the engine would run them eagerly)
        live = [s for s in live if s.length <= width * 16 and len(s.blocks) <= width]


def test_decode_rows_fit_rules():
    rows = _DecodeRows(4, 2, 7, "cpu")
    short = _seq(1, list(range(20)), blocks=[1, 2])
    long = _seq(2, list(range(40)), blocks=[1, 2, 3])
    assert rows.fits([short], 16) and not rows.fits([long], 16)
    assert not rows.fits([short] * 5, 16)


def test_decode_rows_resend_a_replaced_block_list():
    """A sequence keeps its row while the steps in between run eagerly (no sync), and its
    block list is replaced meanwhile (swap-out and swap-in, or a recompute): the next sync
    must send the new ids, not only the entries past the old count."""
    rows = _DecodeRows(4, 6, 99, "cpu")
    a = _seq(1, list(range(40)), blocks=[1, 2, 3])
    b = _seq(2, list(range(20)), blocks=[4, 5])
    rows.sync([a, b])
    a.blocks = [10, 11, 12]                       # swapped out and back into other blocks
    b.blocks = [7]                                # recomputed into a shorter list
    b.tokens = b.tokens[:10]
    rows.forget_tokens()                          # the eager steps in between
    rows.sync([a, b])
    tok, ctx, tab = _expect(rows, [a, b], rows.tok.clone())
    assert torch.equal(rows.table, tab) and torch.equal(rows.ctx, ctx)
    assert rows.table[rows.row_of()[id(b)]].tolist() == [7, 99, 99, 99, 99, 99]
    # growth by append on the same list is still sent incrementally
    a.blocks.append(13)
    a.tokens += [0] * 16
    rows.sync([a, b])
    assert rows.table[rows.row_of()[id(a)]].tolist() == [10, 11, 12, 13, 99, 99]
