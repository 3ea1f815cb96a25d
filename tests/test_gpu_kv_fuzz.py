"""GPU parity of the device-resident KV caches (zwg_kv_*) over seeded random shapes and append
sequences, against oracle/kv.py bit for bit.

Each case draws a layout (row-major decoder cache, or Qwen2's transposed key cache with rotary
positions on k and q), a head dim, KV heads and GQA group, a cache length (a multiple of 4 for
the transposed layout), a rotary base, and a sequence of appends of random lengths until the
cache is full or the draw stops, into a random layer and sequence.  Appends are copies and the
rotations use the reference's f32 tables and rounding (src/decoder.zig:182-183,
src/llm.zig:182-190), so cache contents and rotated q must match the oracle exactly.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import kv as okv

pytestmark = pytest.mark.gpu

N_CASES = 24


@pytest.fixture(scope="module")
def torch():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    return torch


@pytest.fixture(scope="module")
def ctx(torch):
    import zwhisper_amd as z

    c = z.Context(0)
    yield c
    c.close()


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


@pytest.mark.parametrize("seed", range(N_CASES))
def test_kv_fuzz(torch, ctx, seed):
    import zwhisper_amd as z

    rng = np.random.default_rng(6200 + seed)
    kt = bool(rng.integers(2))
    d = int(rng.choice([32, 64, 128]))
    hkv = int(rng.choice([1, 2, 4]))
    group = int(rng.choice([1, 2, 7]))
    h = hkv * group
    n_ctx = 4 * int(rng.integers(1, 300))
    n_layer, n_seq = int(rng.integers(1, 3)), int(rng.integers(1, 3))
    base = float(rng.choice([1.0e4, 1.0e6]))
    kvw, ne = hkv * d, h * d
    print(f"case {seed}: {'KT' if kt else 'ROW'} d {d} hkv {hkv} h {h} n_ctx {n_ctx} "
          f"layers {n_layer} seqs {n_seq} base {base:g}", flush=True)
    layout = z.KV_KT if kt else z.KV_ROW
    extra = {"rope_base": base} if kt else {}
    cos, sin = okv.rope_tables(n_ctx, d, base) if kt else (None, None)
    with z.KVCache(ctx, n_layer, n_seq, n_ctx, hkv, d, layout, **extra) as kv:
        ref = {}
        fill = {}
        for (l, s) in [(l, s) for l in range(n_layer) for s in range(n_seq)]:
            ref[(l, s)] = (np.zeros(hkv * d * n_ctx if kt else n_ctx * kvw, np.float32),
                           np.zeros(n_ctx * kvw, np.float32))
            fill[(l, s)] = 0
        for step in range(int(rng.integers(1, 9))):
            l, s = int(rng.integers(n_layer)), int(rng.integers(n_seq))
            pos = fill[(l, s)]
            if pos == n_ctx:
                continue
            n = int(min(n_ctx - pos, rng.choice([1, 1, 2, 7, 33, 256, n_ctx])))
            k = rng.standard_normal((n, kvw)).astype(np.float32)
            v = rng.standard_normal((n, kvw)).astype(np.float32)
            if kt:
                q = rng.standard_normal((n, ne)).astype(np.float32)
                qd = _dev(torch, q)
                kv.append(l, s, pos, _dev(torch, k), _dev(torch, v), qd, h, ne)
                okv.llm_append(q, k, v, n, pos, h, hkv, d, ne, ref[(l, s)][0], ref[(l, s)][1], n_ctx, cos, sin)
                torch.cuda.synchronize()
                assert np.array_equal(qd.cpu().numpy(), q), f"q rotation, step {step} at {pos}"
            else:
                kv.append(l, s, pos, _dev(torch, k), _dev(torch, v))
                okv.append_rows(ref[(l, s)][0], kvw, pos, k, n)
                okv.append_rows(ref[(l, s)][1], kvw, pos, v, n)
            fill[(l, s)] = pos + n
        torch.cuda.synchronize()
        for key, (rk, rv) in ref.items():
            gk, gv = kv.read(*key)
            assert np.array_equal(gk, rk), f"k cache {key}"
            assert np.array_equal(gv, rv), f"v cache {key}"
