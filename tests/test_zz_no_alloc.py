"""vkml_attend_step_noalloc, the decode-attention step that allocates
nothing (its chunk partials and statistics in the library's own device
scratch), against vkml_attend_step with a workspace of its own: the same
caches, outputs and Q8_0 codes, bit for bit, on two calls in a row, the
second smaller than the first (so it runs over what the first left in the
scratch), and a clean error past the scratch's size."""
import math

import numpy as np
import pytest

from vkml_amd import hip as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    H.init()
    yield
    H.synchronize()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def run_pair(hd, heads, kvh, cap, pos, kv_type, seed):
    """One step through each entry point on identical copies of the caches;
    returns the two results (caches, output, codes, scales) as host arrays."""
    rng = np.random.default_rng(seed)
    chunks = (cap + 127) // 128
    dt = np.uint16 if kv_type == H.F16 else np.float32
    prior = rng.standard_normal((2, kvh, cap, hd)).astype(np.float32)
    caches = [prior[i].astype(np.float16).view(np.uint16) if kv_type == H.F16 else prior[i] for i in range(2)]
    qkv = H.to_device(rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32))
    # a table of cos/sin pairs of the right shape: values need not be a real table
    tab = H.to_device(rng.uniform(-1, 1, (cap, hd // 2, 2)).astype(np.float32))
    prm = H.AttendStepParams(heads, kvh, hd, cap, 0, pos, kv_type, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0)
    results = []
    for noalloc in (True, False):
        kc, vc = H.to_device(caches[0]), H.to_device(caches[1])
        out, vals, scs = H.empty(heads * hd * 4), H.empty(heads * hd), H.empty(heads * hd // 32 * 4)
        if noalloc:
            H.call("vkml_attend_step_noalloc", prm, qkv.p, tab.p, kc.p, vc.p, out.p, vals.p, scs.p, None)
        else:
            part, stats = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
            H.call("vkml_attend_step", prm, qkv.p, tab.p, kc.p, vc.p, part.p, stats.p, out.p, vals.p, scs.p, None)
        H.synchronize()
        results.append((kc.download(dt, caches[0].shape), vc.download(dt, caches[1].shape),
                        out.download(np.float32, (heads, hd)), vals.download(np.uint8, (heads * hd,)),
                        scs.download(np.float32, (heads * hd // 32,))))
    return results


def test_noalloc_matches_the_workspace_entry_point_on_two_calls():
    # cfg5's attention at a 4k cache, then a smaller call (fewer heads and
    # chunks) over the scratch the first one left
    for hd, heads, kvh, cap, pos, kv_type, seed in ((128, 32, 8, 4352, 4200, H.F16, 1), (64, 8, 2, 300, 170, H.F32, 2)):
        print(f"noalloc case hd={hd} heads={heads} kv_heads={kvh} cap={cap} pos={pos}", flush=True)
        a, b = run_pair(hd, heads, kvh, cap, pos, kv_type, seed)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        assert np.array_equal(bits(a[2]), bits(b[2]))
        assert np.array_equal(a[3], b[3])
        assert np.array_equal(bits(a[4]), bits(b[4]))
        assert np.all(np.isfinite(a[2]))


def test_noalloc_rejects_more_than_its_scratch():
    # 64 heads of 256 at 1024 chunks: 64 MiB of partials
    prm = H.AttendStepParams(64, 8, 256, 1024 * 128, 0, 0, H.F16, 1024, 0, 1, 0.0625, 0.0)
    dummy = H.empty(256)
    with pytest.raises(H.VkmlError, match="scratch"):
        H.call("vkml_attend_step_noalloc", prm, dummy.p, dummy.p, dummy.p, dummy.p, dummy.p, dummy.p, dummy.p, None)
