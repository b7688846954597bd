"""GPU parity: decode-step sampling (``moss_sample_topk``, ``moss_compose_next_ids``) vs the oracle.

Bars: argmax, top-k selection and the composed ids are exact; a sampled index equals the oracle's
draw with the same Philox uniform, except where the oracle's target ``u * sum(kept)`` lies within
1e-5 (relative) of a cumulative-probability boundary, where the neighbouring kept index is accepted
(the kernel's expf and summation order differ from numpy's in the last bits).
"""
import numpy as np
import pytest
import torch

from oracle import sampling as os_

pytestmark = pytest.mark.gpu


def _logits(rows, stride, seed, scale=3.0, ties=False):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, stride, generator=g) * scale).bfloat16()
    if ties:
        x[:, 10] = x[:, 500] = x.max() + 1
    return x


def _check_draw(got, row_logits, temperature, top_k, top_p, u, what):
    ref, probs, idx = os_.sample_row(row_logits, temperature, top_k, top_p, u)
    if got == ref:
        return
    kept = probs > 0
    assert kept[list(idx).index(got)], f"{what}: drew a removed index"
    cdf = np.cumsum(probs.astype(np.float64))
    target = float(u) * float(probs.sum(dtype=np.float64))
    gap = np.min(np.abs(cdf[kept] - target))
    assert gap <= 1e-5 * max(target, 1e-30), f"{what}: {got} vs {ref}, target {target} not at a boundary"


@pytest.mark.parametrize("ties", [False, True])
def test_greedy_is_first_argmax(dev, ties):
    from moss_tts._runtime import sampling

    x = _logits(32, 1025, 1, ties=ties)
    got = sampling.sample_topk(x.to(dev), 0.0, 25, 0.8, vocab=1024).cpu().numpy()
    ref = np.argmax(x[:, :1024].float().numpy(), axis=1)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("temperature,top_k,top_p,rows,stride,vocab", [(1.7, 25, 0.8, 32, 1025, 1024),
                                                                       (1.5, 2, 1.0, 1, 2, 2),
                                                                       (1.0, 64, 0.95, 4, 2048, 2048),
                                                                       (0.7, 1, 0.5, 8, 300, 300)])
def test_sampling_matches_oracle_draws(dev, temperature, top_k, top_p, rows, stride, vocab):
    from moss_tts._runtime import sampling

    print(f"sample_topk T={temperature} k={top_k} p={top_p} rows={rows} vocab={vocab}", flush=True)
    x = _logits(rows, stride, 2)
    xd = x.to(dev)
    for position in (0, 7, 2047, 2**33 + 5):
        pos = torch.tensor([position], dtype=torch.int64, device=dev)
        for seed in (0, 12345678901234):
            got = sampling.sample_topk(xd, temperature, top_k, top_p, seed=seed, position=pos, salt=3,
                                       vocab=vocab).cpu().numpy()
            for r in range(rows):
                u = os_.uniform(seed, position, r, 3)
                _check_draw(int(got[r]), x[r, :vocab].float().numpy(), temperature, top_k, top_p, u,
                            f"pos {position} seed {seed} row {r}")


@pytest.mark.parametrize("greedy", [False, True])
def test_sample_pair_equals_two_calls(dev, greedy):
    """One launch for two row sets (the decode step's text row and 32 audio rows) returns what the
    two separate sample_topk calls return, over positions and seeds (the sets restart their row
    numbers, so each keeps its own random stream)."""
    from moss_tts._runtime import sampling

    text = _logits(1, 2, 5).to(dev).view(-1)
    audio = _logits(32, 1025, 6).to(dev)
    for position in (0, 9, 2047, 2**33 + 5):
        pos = torch.tensor([position], dtype=torch.int64, device=dev)
        for seed in (0, 987654321):
            print(f"sample pair greedy={greedy} position={position} seed={seed}", flush=True)
            sb = sampling.seed_buffer(seed, dev)
            t_ref = sampling.sample_topk(text, 0.0 if greedy else 1.5, 2, 1.0, seed=sb, position=pos, salt=1)
            a_ref = sampling.sample_topk(audio, 0.0 if greedy else 1.7, 25, 0.8, seed=sb, position=pos, salt=0,
                                         vocab=1024)
            t_out = torch.full((1,), -1, dtype=torch.int64, device=dev)
            a_out = torch.full((32,), -1, dtype=torch.int64, device=dev)
            sampling.sample_topk_pair(
                dict(logits=text, temperature=0.0 if greedy else 1.5, top_k=2, top_p=1.0, salt=1, out=t_out),
                dict(logits=audio, temperature=0.0 if greedy else 1.7, top_k=25, top_p=0.8, salt=0, vocab=1024,
                     out=a_out),
                seed=sb, position=pos)
            assert torch.equal(t_out, t_ref) and torch.equal(a_out, a_ref)


def _candidate_count(row_logits: np.ndarray, temperature: float, top_k: int) -> int:
    """How many keys the kernel's threshold keeps: those >= the k-th largest per-lane maximum
    (lane l holds indices l + 64 j).  Tells which selection branch a case exercises."""
    v = (row_logits.astype(np.float32) / np.float32(temperature)).astype(np.float64)
    order = np.lexsort((np.arange(v.size), -v))          # rank 0 = largest key
    rank = np.empty(v.size, dtype=np.int64)
    rank[order] = np.arange(v.size)
    lane_best = [rank[lane::64].min() for lane in range(min(64, v.size))]
    thresh = sorted(lane_best)[top_k - 1]
    return int((rank <= thresh).sum())


def _pattern(name: str, rows: int, stride: int):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(rows, stride, generator=g)
    if name == "lanes":           # the largest values all sit in lanes 0..4: more than 64 candidates
        for lane in range(5):
            x[:, lane::64] += 20.0
    elif name == "equal":         # one value everywhere: the order is the index order
        x[:] = 1.25
    elif name == "neg_inf":       # all but 30 entries masked
        keep = x.clone()
        x[:] = -float("inf")
        x[:, 3::37] = keep[:, 3::37]
    return x.bfloat16()


@pytest.mark.parametrize("name,top_k,top_p,vocab,branch", [("lanes", 25, 0.8, 1024, "rounds"),
                                                          ("lanes", 64, 0.95, 1024, "rounds"),
                                                          ("equal", 25, 0.8, 1024, "rank"),
                                                          ("neg_inf", 25, 0.9, 1024, "rank"),
                                                          ("random", 40, 1.0, 40, "rank")])
def test_sampling_selection_branches(dev, name, top_k, top_p, vocab, branch):
    """Both selection branches (rank among <= 64 candidates; rounds of argmax over more) draw the
    oracle's index; the branch taken is predicted on the CPU from the same threshold."""
    from moss_tts._runtime import sampling

    print(f"sample_topk pattern={name} k={top_k} vocab={vocab}", flush=True)
    rows, stride, temperature = 4, 1025, 1.7
    x = _pattern(name, rows, stride)
    for r in range(rows):
        c = _candidate_count(x[r, :vocab].float().numpy(), temperature, top_k)
        assert (c > 64) == (branch == "rounds"), (name, r, c)
    xd = x.to(dev)
    for position in (0, 7, 2047):
        pos = torch.tensor([position], dtype=torch.int64, device=dev)
        got = sampling.sample_topk(xd, temperature, top_k, top_p, seed=77, position=pos, salt=0,
                                   vocab=vocab).cpu().numpy()
        for r in range(rows):
            _check_draw(int(got[r]), x[r, :vocab].float().numpy(), temperature, top_k, top_p,
                        os_.uniform(77, position, r, 0), f"{name} pos {position} row {r}")
    greedy = sampling.sample_topk(xd, 0.0, 25, 0.8, vocab=vocab).cpu().numpy()
    assert np.array_equal(greedy, np.argmax(x[:, :vocab].float().numpy(), axis=1))


def test_sampling_frequencies(dev):
    """Across 2000 positions one row's draws follow the kept probabilities (chi-square bound)."""
    from moss_tts._runtime import sampling

    x = _logits(1, 64, 3, scale=1.0)
    _, probs, idx = os_.sample_row(x[0].float().numpy(), 1.0, 8, 0.9, 0.0)
    p = probs / probs.sum()
    n = 2000
    counts = np.zeros(len(p))
    xd = x.to(dev)
    pos = torch.zeros(1, dtype=torch.int64, device=dev)
    outs = []
    for t in range(n):
        pos.fill_(t)
        outs.append(sampling.sample_topk(xd, 1.0, 8, 0.9, seed=99, position=pos))
    for o in torch.cat(outs).cpu().numpy():
        counts[list(idx).index(int(o))] += 1
    keep = p > 0
    assert counts[~keep].sum() == 0
    chi2 = (((counts - n * p)[keep] ** 2) / (n * p[keep])).sum()
    assert chi2 < 30.0


@pytest.mark.parametrize("audio_length,delay_length,text_index", [(32, -1, 0), (5, -1, 1), (32, 0, 0), (32, 7, 1),
                                                                  (32, 32, 0), (3, 1, 1)])
def test_compose_next_ids(dev, audio_length, delay_length, text_index):
    from moss_tts._runtime import sampling

    audio = torch.arange(100, 132, dtype=torch.int64, device=dev)
    text_ids = torch.tensor([151656, 151662], dtype=torch.int64, device=dev)
    out = sampling.compose_next_ids(torch.tensor([text_index], device=dev), audio, text_ids,
                                    torch.tensor([audio_length], device=dev), torch.tensor([delay_length], device=dev),
                                    delay_slot_id=151662, audio_end_id=151653).cpu().numpy()
    ref = os_.compose_next_ids(text_index, np.arange(100, 132), [151656, 151662], audio_length, delay_length,
                               151662, 151653)
    assert np.array_equal(out, ref)


@pytest.mark.parametrize("greedy", [True, False])
def test_decode_step_next_ids(dev, greedy):
    """The captured step's next ids equal the oracle's sampling of that step's own logits."""
    from moss_tts._runtime.decode import CODEBOOKS, DecodeStepG32

    print(f"decode next ids greedy={greedy}", flush=True)
    eng = DecodeStepG32.random(1, max_length=128, device=dev, seed=5, text_vocab=256, greedy=greedy, sample_seed=42)
    eng.capture()
    ids = torch.tensor([[17] + [3] * 32], dtype=torch.int64)
    for position, audio_length, delay_length in ((5, 32, -1), (9, 12, -1), (20, 32, 4)):
        nxt = eng.decode(ids, position, audio_length, delay_length).view(-1).cpu().numpy()
        logits = eng.logits.float().cpu().numpy()
        stride, n_audio = eng.audio_stride, CODEBOOKS * eng.audio_stride
        audio = logits[:n_audio].reshape(CODEBOOKS, stride)[:, :1024]
        text = logits[n_audio:n_audio + 2]
        if greedy:
            t_idx = int(np.argmax(text))
            a_idx = np.argmax(audio, axis=1)
        else:
            t_idx = os_.sample_row(text, 1.5, 2, 1.0, os_.uniform(42, position, 0, 1))[0]
            a_idx = np.array([os_.sample_row(audio[c], 1.7, 25, 0.8, os_.uniform(42, position, c, 0))[0]
                              for c in range(CODEBOOKS)])
        ref = os_.compose_next_ids(t_idx, a_idx, eng.text_ids_host, audio_length, delay_length,
                                   eng.text_ids_host[1], eng.audio_end_id)
        if greedy:
            assert np.array_equal(nxt, ref)
        else:
            # the text token and masked channels are exact; sampled codes obey the draw bar
            assert nxt[0] == ref[0]
            for c in range(CODEBOOKS):
                valid = c < audio_length and (delay_length < 0 or c >= delay_length)
                if not valid:
                    assert nxt[1 + c] == 1024
                else:
                    _check_draw(int(nxt[1 + c]), audio[c], 1.7, 25, 0.8, os_.uniform(42, position, c, 0),
                                f"pos {position} channel {c}")


START, GEN, DELAY = 151652, 151656, 151662


@pytest.mark.parametrize("text,delay,with_outputs", [(GEN, -1, True), (DELAY, -1, True), (DELAY, 4, False),
                                                     (GEN, 7, True), (START, -1, True), (42, -1, True),
                                                     (42, 0, False)])
def test_advance_step_matches_oracle(dev, text, delay, with_outputs):
    from moss_tts._runtime import sampling

    nxt = torch.tensor([text] + list(range(500, 532)), dtype=torch.int64, device=dev)
    ids = torch.zeros(33, dtype=torch.int64, device=dev)
    pos = torch.tensor([77], dtype=torch.int64, device=dev)
    length = torch.tensor([5], dtype=torch.int64, device=dev)
    dl = torch.tensor([delay], dtype=torch.int64, device=dev)
    history = torch.full((4, 33), -9, dtype=torch.int64, device=dev) if with_outputs else None
    status = torch.full((4,), -9, dtype=torch.int64, device=dev) if with_outputs else None
    sampling.advance_step(nxt, ids, pos, length, dl, step=2, history=history, status=status, audio_start_id=START,
                          gen_slot_id=GEN, delay_slot_id=DELAY)
    r_ids, r_pos, r_len, r_delay, r_status = os_.advance_state(nxt.cpu().numpy(), 77, 5, delay, audio_start_id=START,
                                                               gen_slot_id=GEN, delay_slot_id=DELAY)
    assert np.array_equal(ids.cpu().numpy(), r_ids)
    assert (int(pos), int(length), int(dl)) == (r_pos, r_len, r_delay)
    if with_outputs:
        h = history.cpu().numpy()
        assert np.array_equal(h[2], r_ids) and (h[[0, 1, 3]] == -9).all()
        assert np.array_equal(status.cpu().numpy(), r_status)


@pytest.mark.parametrize("delay,prefixes", [(-1, True), (0, True), (-1, False)])
def test_first_audio_graph_equals_sequential_steps(dev, delay, prefixes):
    """32 steps in one graph (device-side advance) give the same next ids, step for step, and the
    same final state as 32 single decode steps with the host-side update; with head prefixes the
    graph computes only the first 8/16/24/32 audio heads, which changes no emitted id."""
    from moss_tts._runtime.decode import CODEBOOKS, DecodeStepG32, FirstAudioGraph

    print(f"first-audio graph delay={delay} head_prefixes={prefixes}", flush=True)
    eng = DecodeStepG32.random(1, max_length=128, device=dev, seed=9, text_vocab=256, sample_seed=7)
    eng.capture()
    burst = FirstAudioGraph(eng, steps=CODEBOOKS, head_prefixes=prefixes)
    first = torch.full((1, 1, 33), 1024, dtype=torch.int64, device=dev)
    first[0, 0, 0] = eng.audio_start_id
    with pytest.raises(RuntimeError, match="Warm"):
        burst.run(first, 40)
    burst.warmup()
    with pytest.raises(ValueError, match="capacity"):
        burst.run(first, 128 - CODEBOOKS + 1)
    with pytest.raises(ValueError, match="audio-start row"):
        burst.run(first.view(1, 33), 40)
    with pytest.raises(ValueError, match="fresh audio"):
        burst.run(first, 40, delay=3)
    start = 40
    hist, status = burst.run(first, start, delay=delay)
    hist = hist.cpu().numpy().copy()
    status = status.cpu().numpy().copy()
    gen, dslot = eng.text_ids_host
    ids, pos, length, d = first, start, 1, delay
    for t in range(CODEBOOKS):
        nxt = eng.decode(ids.view(1, 33), pos, audio_length=length, delay_length=d)
        row = nxt.view(-1).cpu().numpy()
        assert np.array_equal(row, hist[t]), f"step {t}"
        _, pos, length, d, st = os_.advance_state(row, pos, length, d, audio_start_id=eng.audio_start_id,
                                                  gen_slot_id=gen, delay_slot_id=dslot)
        ids = nxt
    assert np.array_equal(status, st)
    assert set(hist[:, 0]) <= {gen, dslot}
    if delay == 0:   # the probe starts the delay counter: every composed text token is the delay slot
        assert (hist[:, 0] == dslot).all() and int(status[2]) == CODEBOOKS


def test_seed_per_request(dev):
    """The sampler reads its key from a device buffer: after capture, a new seed changes the draws
    of the replayed graph (they follow the oracle's Philox uniforms for that seed), the same seed
    reproduces them, and the first-audio graph takes a per-run seed the same way."""
    from moss_tts._runtime.decode import CODEBOOKS, DecodeStepG32, FirstAudioGraph

    print("per-request seed", flush=True)
    eng = DecodeStepG32.random(1, max_length=128, device=dev, seed=5, text_vocab=256, sample_seed=7)
    eng.capture()
    ids = torch.tensor([[17] + [3] * 32], dtype=torch.int64)
    a = eng.decode(ids, 5, seed=1).view(-1).cpu().numpy()
    b = eng.decode(ids, 5, seed=2).view(-1).cpu().numpy()
    assert eng.seed == 2
    logits = eng.logits.float().cpu().numpy()
    audio = logits[:CODEBOOKS * eng.audio_stride].reshape(CODEBOOKS, eng.audio_stride)[:, :1024]
    for c in range(CODEBOOKS):
        _check_draw(int(b[1 + c]), audio[c], 1.7, 25, 0.8, os_.uniform(2, 5, c, 0), f"seed 2 channel {c}")
    again = eng.decode(ids, 5, seed=1).view(-1).cpu().numpy()
    assert np.array_equal(a, again)
    assert not np.array_equal(a[1:], b[1:])
    eng.seed = (1 << 64) - 3          # the full 64-bit range round-trips through the int64 buffer
    assert eng.seed == (1 << 64) - 3
    burst = FirstAudioGraph(eng, steps=8)
    burst.warmup()
    first = torch.full((1, 1, 33), 1024, dtype=torch.int64, device=dev)
    first[0, 0, 0] = eng.audio_start_id
    h3 = burst.run(first, 40, seed=3)[0].cpu().numpy().copy()
    h4 = burst.run(first, 40, seed=4)[0].cpu().numpy().copy()
    h3b = burst.run(first, 40, seed=3)[0].cpu().numpy().copy()
    assert np.array_equal(h3, h3b) and not np.array_equal(h3, h4)
