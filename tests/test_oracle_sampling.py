"""Pins the sampling oracle (``oracle/sampling.py``) on the CPU.

* Philox4x32-10 equals the published known-answer vectors of the Random123 distribution.
* The top-k set and order equal ``torch.topk`` on distinct values; the greedy path equals
  ``torch.argmax`` (first maximal index) including ties.
* The kept probabilities equal ``torch.softmax`` of the top-k values with the reference's top-p
  mask (``cumsum - p > top_p``), restated with torch ops.
* The u-inversion draws each index with its probability: frequencies over 40,000 Philox draws lie
  within a chi-square bound of the exact probabilities, and so do ``torch.multinomial``'s.
* The next-id composition equals a restatement of the reference's two ``torch.where`` lines.
"""
import numpy as np
import pytest
import torch

from oracle import sampling as s


@pytest.mark.parametrize("ctr,key,expected", [
    ((0, 0, 0, 0), (0, 0), "6627e8d5 e169c58d bc57ac4c 9b00dbd8"),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, "408f276d 41c83b0e a20bc7c6 6d5451fd"),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     "d16cfe09 94fdcceb 5001e420 24126ea1"),
])
def test_philox_known_answers(ctr, key, expected):
    assert " ".join(f"{v:08x}" for v in s.philox4x32_10(ctr, key)) == expected


def test_topk_and_argmax_match_torch():
    g = torch.Generator().manual_seed(0)
    for _ in range(20):
        x = torch.randn(1024, generator=g)
        idx, vals = s.topk(x.numpy(), 25)
        tv, ti = torch.topk(x, 25)
        assert np.array_equal(idx, ti.numpy()) and np.array_equal(vals, tv.numpy())
    # greedy with ties: the first maximal index, as torch.argmax documents
    x = torch.zeros(1024).bfloat16()
    x[[7, 300, 900]] = 3.0
    assert s.sample_row(x.float().numpy(), 0.0, 25, 0.8, 0.5)[0] == int(torch.argmax(x.float())) == 7


def test_probabilities_match_the_reference_formula():
    g = torch.Generator().manual_seed(1)
    logits = (torch.randn(1024, generator=g) * 3).bfloat16().float()
    _, probs, idx = s.sample_row(logits.numpy(), 1.7, 25, 0.8, 0.3)
    values, indexes = torch.topk(logits / 1.7, 25)
    p = values.softmax(-1)
    remove = p.cumsum(-1) - p > 0.8
    p = p.masked_fill(remove, 0)
    assert np.array_equal(idx, indexes.numpy())
    assert np.allclose(probs, p.numpy(), rtol=1e-6, atol=1e-7)
    assert (probs == 0).sum() == int(remove.sum())


def test_inversion_draws_the_probabilities():
    g = torch.Generator().manual_seed(2)
    logits = (torch.randn(64, generator=g) * 2).bfloat16().float().numpy()
    _, probs, idx = s.sample_row(logits, 1.0, 8, 0.9, 0.0)
    p = probs / probs.sum()
    n = 40000
    counts = {}
    for t in range(n):
        j = s.sample_row(logits, 1.0, 8, 0.9, s.uniform(1234, t, 0))[0]
        counts[j] = counts.get(j, 0) + 1
    obs = np.array([counts.get(int(i), 0) for i in idx])
    assert obs.sum() == n and all(obs[p == 0] == 0)
    keep = p > 0
    chi2 = (((obs - n * p)[keep] ** 2) / (n * p[keep])).sum()
    assert chi2 < 30.0, chi2                          # 8 cells: p(chi2 > 30) < 1e-4
    tm = torch.multinomial(torch.from_numpy(probs), n, replacement=True, generator=torch.Generator().manual_seed(3))
    tobs = np.bincount(tm.numpy(), minlength=len(p))
    assert all(tobs[~keep] == 0)
    chi2_t = (((tobs - n * p)[keep] ** 2) / (n * p[keep])).sum()
    assert chi2_t < 30.0, chi2_t


@pytest.mark.parametrize("audio_length,delay_length", [(32, -1), (5, -1), (32, 0), (32, 7), (32, 32), (3, 1)])
def test_compose_matches_the_reference_where_lines(audio_length, delay_length):
    text_ids = torch.tensor([151656, 151662])
    audio = torch.arange(100, 132)
    text_index = torch.tensor(1)
    tok = text_ids[text_index]
    tok = torch.where(torch.tensor(delay_length) >= 0, 151662, tok)
    tok = torch.where(torch.tensor(delay_length) == 32, 151653, tok)
    channels = torch.arange(32)
    valid = (channels < audio_length) & ((torch.tensor(delay_length) < 0) | (channels >= delay_length))
    ref = torch.cat([tok.view(1), torch.where(valid, audio, 1024)]).numpy()
    got = s.compose_next_ids(1, audio.numpy(), text_ids.numpy(), audio_length, delay_length, 151662, 151653)
    assert np.array_equal(got, ref)


START, GEN, DELAY, END = 151652, 151656, 151662, 151653


@pytest.mark.parametrize("first_delay", [None, 0, 5, 20])
def test_advance_state_closed_forms(first_delay):
    """Over a run of in-audio steps: the delay counter after step t is t - t0 + 1 once the first
    delay-slot token appeared at t0 (else -1), the audio length counts the start / gen / delay
    tokens, and the position counts steps."""
    pos, length, delay = 100, 1, -1
    for t in range(40):
        tok = DELAY if first_delay is not None and t >= first_delay else GEN
        ids = np.array([tok] + [7] * 32)
        _, pos, length, delay, status = s.advance_state(ids, pos, length, delay, audio_start_id=START,
                                                        gen_slot_id=GEN, delay_slot_id=DELAY)
        assert pos == 101 + t and length == 2 + t
        assert delay == (t - first_delay + 1 if first_delay is not None and t >= first_delay else -1)
        assert list(status) == [tok, length, delay, pos]
    # other text tokens (an ordinary text id) leave the audio length alone
    _, _, length2, delay2, _ = s.advance_state(np.array([42] * 33), 0, 3, -1, audio_start_id=START, gen_slot_id=GEN,
                                               delay_slot_id=DELAY)
    assert (length2, delay2) == (3, -1)


def test_advance_then_compose_ends_audio_after_32_delay_steps():
    """Composition and state update together: once the text head first picks the delay slot, the
    composed text token is the delay slot until, 32 steps later, the audio end."""
    text_ids = np.array([GEN, DELAY])
    pos, length, delay = 0, 1, -1
    first = 3
    emitted = []
    for t in range(40):
        text_index = 1 if t == first else 0       # the head asks for the delay slot once, at step 3
        nxt = s.compose_next_ids(text_index, np.arange(32), text_ids, length, delay, DELAY, END)
        emitted.append(int(nxt[0]))
        _, pos, length, delay, _ = s.advance_state(nxt, pos, length, delay, audio_start_id=START, gen_slot_id=GEN,
                                                   delay_slot_id=DELAY)
    assert emitted[:first] == [GEN] * first
    assert emitted[first:first + 32] == [DELAY] * 32
    assert emitted[first + 32] == END
