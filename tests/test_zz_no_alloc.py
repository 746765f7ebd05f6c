"""dwim_attention_noalloc (no counterpart in the reference: dwim_attention for
callers that cannot allocate) against dwim_attention through the C ABI: the
same bits, on two calls in a row, the second smaller than the first, then a
batch on the matrix-core path and decode calls on the matrix-core decode
pass; and a call past its fixed scratch array is refused with a clear
error."""
import numpy as np
import pytest

from dwim_amd import device as D


def _case(gpu, rng, n, pos, heads, kvh, hd):
    kv = (pos + n) * kvh * hd
    kc, vc = gpu.alloc_cache(kv), gpu.alloc_cache(kv)
    gpu.store(kc, 0, gpu.buffer(rng.standard_normal(kv).astype(np.float32)))
    gpu.store(vc, 0, gpu.buffer(rng.standard_normal(kv).astype(np.float32)))
    q = gpu.buffer(rng.standard_normal(n * heads * hd).astype(np.float32))
    return kc, vc, q


@pytest.mark.gpu
def test_noalloc_attention_equals_attention():
    gpu = D.Hip(0)
    rng = np.random.default_rng(7)
    # one token over the VALU pass; a few tokens over it (head_dim 128); a
    # batch through the flash kernel; one token and a verify-sized group past
    # 6144 positions through the decode pass on the matrix cores
    for n, pos, heads, kvh, hd in ((1, 4095, 24, 4, 256), (3, 100, 4, 2, 128), (20, 70, 24, 4, 256),
                                   (1, 5, 6, 6, 64), (1, 9000, 24, 4, 256), (4, 20000, 24, 4, 256)):
        print(f"noalloc case n={n} pos={pos} heads={heads}/{kvh} hd={hd}", flush=True)
        kc, vc, q = _case(gpu, rng, n, pos, heads, kvh, hd)
        want, got = gpu.alloc(n * heads * hd), gpu.alloc(n * heads * hd)
        gpu.attention(want, q, kc, vc, pos, heads, hd, kvh)
        gpu.attention_noalloc(got, q, kc, vc, pos, heads, hd, kvh)
        a, b = gpu.read(want), gpu.read(got)
        assert np.all(np.isfinite(a))
        assert a.tobytes() == b.tobytes()
    gpu.close()


@pytest.mark.gpu
def test_noalloc_attention_refuses_more_than_its_scratch():
    gpu = D.Hip(0)
    n, pos, heads, kvh, hd = 2, 180000, 24, 4, 256
    kv = (pos + n) * kvh * hd
    kc, vc = gpu.alloc_cache(kv), gpu.alloc_cache(kv)
    q, out = gpu.alloc(n * heads * hd), gpu.alloc(n * heads * hd)
    with pytest.raises(D.DwimError, match="scratch array"):
        gpu.attention_noalloc(out, q, kc, vc, pos, heads, hd, kvh)
    # a batch's expanded cache: 64 KiB per 32 positions and key/value head,
    # 8192 positions at 4 heads; 16 tokens at 8180 pass that
    n, pos = 16, 8180
    q, out = gpu.alloc(n * heads * hd), gpu.alloc(n * heads * hd)
    with pytest.raises(D.DwimError, match="expanded cache"):
        gpu.attention_noalloc(out, q, kc, vc, pos, heads, hd, kvh)
    gpu.close()
