"""GPU: the streaming-read measurement kernel (``moss_stream_read``) reads exactly the requested
bytes: each wave's XOR of the 32-bit words it read equals the same XOR on the CPU, for a single
chunk, a workgroup's 16 KiB, a ragged last workgroup and the 29,130,752 bytes of the K=4096
N=12288 GEMV (thread t of workgroup b reads 16-byte chunks 1024 b + 256 u + t, u < 4)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

WG_BYTES = 16 << 10


@pytest.mark.parametrize("nbytes", [16, WG_BYTES, WG_BYTES + 16, 3 * WG_BYTES - 48, 29130752])
def test_stream_read_xor(dev, nbytes):
    from moss_tts._runtime import native

    print(f"stream read {nbytes} bytes", flush=True)
    g = torch.Generator().manual_seed(nbytes)
    src = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), generator=g, dtype=torch.int32)
    words = int(native.lib().moss_stream_read_words(nbytes))
    wgs = -(-nbytes // WG_BYTES)
    assert words == 4 * wgs
    out = torch.full((words,), -1, dtype=torch.int32, device=dev)
    d = src.to(dev)
    native.call("moss_stream_read", native.ptr(d), nbytes, native.ptr(out), native.stream_of(d))
    torch.cuda.synchronize()
    pad = np.zeros(wgs * WG_BYTES // 4, dtype=np.uint32)
    pad[:src.numel()] = src.numpy().view(np.uint32)
    # [workgroup, load u, wave w, lane, 4 words] -> XOR over u, lane and word per (workgroup, wave)
    ref = np.bitwise_xor.reduce(pad.reshape(wgs, 4, 4, 64 * 4).transpose(0, 2, 1, 3).reshape(wgs * 4, -1), axis=1)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref)
