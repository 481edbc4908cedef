"""GPU: ornith_hip_matvec_noalloc (the entry point that allocates nothing; its
scratch is a fixed device array) against ornith_hip_matvec, through the C
ABI. Bar: bit-exact, on two calls in a row (the second on a smaller input, so
stale scratch contents from the first would show), for every weight type and
the integer and f32-fallback paths; sizes above the scratch limit are
rejected with an error."""
import numpy as np
import pytest

import clibs
from clibs import F32, IQ2_XXS, Q4_K, Q6_K, Q8_0

pytestmark = pytest.mark.gpu


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0, IQ2_XXS, F32], ids=["Q4_K", "Q6_K", "Q8_0", "IQ2_XXS", "F32"])
def test_noalloc_matvec_equals_matvec(hip_ctx, orc, t):
    # first call: a large matrix and two columns; second: a smaller one
    for k, (n, out, tn) in enumerate(((2048, 4096, 2), (512, 300, 1))):
        w = clibs.gauss(40 + k, f"na.{t}.{n}.{out}", n * out, 0.02)
        enc = clibs.quantize(orc, t, w) if t != F32 else w.view(np.uint8)
        W = hip_ctx.upload("na", t, enc, (n, out))
        x = np.concatenate([clibs.gauss(50 + k + c, f"nx.{n}.{c}", n, 1.0) for c in range(tn)])
        ref = W.matvec(x)
        got = W.matvec_noalloc(x)
        assert np.array_equal(u32(got), u32(ref)), (k, np.nonzero(u32(got) != u32(ref))[0][:8])
        W.free()


def test_noalloc_rejects_beyond_limit(hip_ctx, orc):
    import ornithology_amd as oa
    # 1,100,000 output rows need more than the 4 MiB scratch (4.4 MB of
    # outputs alone); the check happens before any device work
    n, out = 256, 1_100_000
    enc = np.zeros(out * clibs.row_bytes(IQ2_XXS, n), np.uint8)
    W = hip_ctx.upload("big", IQ2_XXS, enc, (n, out))
    with pytest.raises(oa.HipError):
        W.matvec_noalloc(np.ones(n, np.float32))
    W.free()
