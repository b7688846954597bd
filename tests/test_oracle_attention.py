"""Pins the attention oracle (``oracle/attention.py``) and the composed decode step's pieces on
the CPU.

* ``decode_attention`` equals a float64 loop restatement (per head: scores, max-subtracted
  softmax, weighted sum) and torch's own ``scaled_dot_product_attention`` in fp32 with the
  KV heads repeated for their 4 query heads; rows after ``position`` never matter.
* ``embedding_sum`` equals its definition (text row, then each codebook row added with a bf16
  rounding after every addition), checked on a case where the rounding order is visible.
"""
import math

import torch

from oracle import attention as oa


def _case(L, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((32, 128), generator=g).bfloat16()
    kc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    return q, kc, vc


def test_decode_attention_matches_float64_loops():
    q, kc, vc = _case(24, 0)
    p = 17
    got = oa.decode_attention(q, kc, vc, p).double()
    for h in (0, 3, 4, 31):
        kv = h // 4
        qh = q[h].double()
        s = [float((qh * kc[0, kv, t].double()).sum()) / math.sqrt(128) for t in range(p + 1)]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        ref = sum(w[t] / z * vc[0, kv, t].double() for t in range(p + 1))
        assert torch.allclose(got[h], ref, atol=1e-5, rtol=1e-5)


def test_decode_attention_matches_torch_sdpa():
    q, kc, vc = _case(96, 1)
    for p in (0, 1, 63, 95):
        k = kc[0, :, : p + 1].float().repeat_interleave(4, dim=0)      # [32, T, 128]
        v = vc[0, :, : p + 1].float().repeat_interleave(4, dim=0)
        ref = torch.nn.functional.scaled_dot_product_attention(q.float()[:, None], k, v)[:, 0]
        assert torch.allclose(oa.decode_attention(q, kc, vc, p), ref, atol=2e-5, rtol=1e-4)


def test_decode_attention_ignores_rows_after_position():
    q, kc, vc = _case(40, 2)
    a = oa.decode_attention(q, kc, vc, 20)
    kc[:, :, 21:] = 1e4
    vc[:, :, 21:] = float("nan")
    assert torch.equal(a, oa.decode_attention(q, kc, vc, 20))


def test_embedding_sum_rounds_after_every_add():
    text = torch.zeros((4, 8), dtype=torch.bfloat16)
    audio = torch.zeros((3, 5, 8), dtype=torch.bfloat16)
    text[2, 0] = 256.0
    audio[0, 1, 0] = 0.75      # 256.75 -> bf16 256 (spacing 2 at 256)
    audio[1, 4, 0] = 0.75      # 256.75 -> 256 again
    audio[2, 3, 0] = 1.0       # 257 -> tie -> 256 (even mantissa)
    ids = torch.tensor([2, 1, 4, 3])
    # rounded after every add: 256; one rounding of the exact sum 258.5 would give 258
    assert float(oa.embedding_sum(ids, text, audio)[0]) == 256.0
    g = torch.Generator().manual_seed(3)
    text = torch.randn((10, 64), generator=g).bfloat16()
    audio = torch.randn((32, 7, 64), generator=g).bfloat16()
    ids = torch.cat([torch.tensor([4]), torch.randint(0, 7, (32,), generator=g)])
    x = text[4].float()
    for c in range(32):
        x = (x + audio[c, int(ids[c + 1])].float()).bfloat16().float()
    assert torch.equal(oa.embedding_sum(ids, text, audio).view(torch.int16), x.bfloat16().view(torch.int16))
