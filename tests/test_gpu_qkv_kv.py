"""GPU parity of zwg_linear_q8w_qkv_kv_dev: a decode step's q/k/v projections over resident int8
weights with the cache append in their final store, against the two calls it replaces
(zwg_linear_q8w_group_dev into rows, then zwg_kv_append_batch), each already checked against f64
and the oracle (tests/test_gpu_linear_q8.py, tests/test_gpu_kv.py).  Bar: q and every
(layer, sequence) cache equal bit for bit -- the fused store takes the same split sums and rotates
them with the same roundings (src/llm.zig:221-238) -- including tokens whose position is outside
the cache (no cache rows, q unrotated) and the rows and sequences the step does not touch.
Shapes: the Whisper small.en decoder step (src/decoder.zig:181-183: row caches, no rotary), the
Qwen2.5-1.5B decode step (src/llm.zig:179-190: transposed keys, rotary base 1e6, GQA 12/2,
d = 128), and a small GQA case with k just above 256 and 33 tokens.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


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


CASES = [
    dict(m=32, k=768, n_head=12, n_head_kv=12, d=64, kt=False, rope=0.0, n_ctx=448, biases=(True, False, True)),
    dict(m=64, k=1536, n_head=12, n_head_kv=2, d=128, kt=True, rope=1e6, n_ctx=4096, biases=(True, True, True)),
    dict(m=33, k=288, n_head=4, n_head_kv=2, d=64, kt=True, rope=1e4, n_ctx=64, biases=(False, True, False)),
]


def weights(rng, n, k):
    import zwhisper_amd as z

    return z.Q8.quantize((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32), n, k)


@pytest.mark.parametrize("c", CASES, ids=["small_en", "qwen15", "gqa_small"])
def test_fused_append_matches_group_then_append(torch, ctx, c):
    import contextlib

    import zwhisper_amd as z
    from zwhisper_amd import _lib

    m, k, d, hq, hk = c["m"], c["k"], c["d"], c["n_head"], c["n_head_kv"]
    rng = np.random.default_rng(m + k + d)
    print(f"qkv+cache m={m} k={k} heads {hq}/{hk} d={d} kt={c['kt']} rope={c['rope']}", flush=True)
    ns = (hq * d, hk * d, hk * d)
    ws = [weights(rng, n, k) for n in ns]
    bs = [torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda() if hb else None
          for n, hb in zip(ns, c["biases"])]
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda()
    pos = rng.integers(0, c["n_ctx"], m).astype(np.int32)
    pos[1] = -1            # outside the cache: no cache rows, q unrotated
    pos[m // 2] = c["n_ctx"]
    pos[2] = c["n_ctx"] - 1
    pos_dev = torch.from_numpy(pos).cuda()
    layout = _lib.KV_KT if c["kt"] else _lib.KV_ROW
    n_seq, seq0, layer = m + 3, 2, 1
    with contextlib.ExitStack() as st:
        rs = [st.enter_context(w.resident(ctx)) for w in ws]
        kv_a = st.enter_context(z.KVCache(ctx, 2, n_seq, c["n_ctx"], hk, d, layout, c["rope"]))
        kv_b = st.enter_context(z.KVCache(ctx, 2, n_seq, c["n_ctx"], hk, d, layout, c["rope"]))
        # the same earlier content in both, so untouched rows are compared too
        for kv in (kv_a, kv_b):
            g = torch.Generator(device="cuda").manual_seed(7)
            for lay in range(2):
                kk = torch.randn(n_seq, hk * d, device="cuda", generator=g)
                vv = torch.randn(n_seq, hk * d, device="cuda", generator=g)
                kv.append_batch(lay, 0, torch.zeros(n_seq, dtype=torch.int32, device="cuda") + 3, kk, vv)
        q_a = torch.full((m, hq * d), float("nan"), device="cuda")
        ctx.linear_q8w_qkv_kv_dev(x, m, rs, bs, q_a, kv_a, layer, seq0, pos_dev)
        q_b = torch.full((m, hq * d), float("nan"), device="cuda")
        k_rows = torch.empty((m, hk * d), device="cuda")
        v_rows = torch.empty((m, hk * d), device="cuda")
        ctx.linear_q8w_group_dev(x, m, rs, bs, [q_b, k_rows, v_rows])
        kv_b.append_batch(layer, seq0, pos_dev, k_rows, v_rows, q=q_b if c["rope"] > 0 else None, n_head=hq,
                          q_stride=hq * d)
        torch.cuda.synchronize()
        assert torch.equal(q_a, q_b)
        for lay in range(2):
            for s in range(n_seq):
                ka, va = kv_a.read(lay, s)
                kb, vb = kv_b.read(lay, s)
                assert np.array_equal(ka, kb) and np.array_equal(va, vb), (lay, s)


def test_fused_append_refusals(torch, ctx):
    import contextlib

    import zwhisper_amd as z

    rng = np.random.default_rng(5)
    with contextlib.ExitStack() as st:
        kv = st.enter_context(z.KVCache(ctx, 1, 70, 64, 2, 64))
        good = [st.enter_context(weights(rng, n, 512).resident(ctx)) for n in (128, 128, 128)]
        short = [st.enter_context(weights(rng, n, 256).resident(ctx)) for n in (128, 128, 128)]
        wide = [st.enter_context(weights(rng, n, 512).resident(ctx)) for n in (128, 192, 128)]
        x = torch.zeros(70 * 512, device="cuda")
        q = torch.zeros(70 * 128, device="cuda")
        pos = torch.zeros(70, dtype=torch.int32, device="cuda")
        with pytest.raises(z.ZwgError, match="at most 64"):
            ctx.linear_q8w_qkv_kv_dev(x, 65, good, None, q, kv, 0, 0, pos)
        with pytest.raises(z.ZwgError, match="above 256"):
            ctx.linear_q8w_qkv_kv_dev(x, 8, short, None, q, kv, 0, 0, pos)
        with pytest.raises(z.ZwgError, match="n_head_kv"):
            ctx.linear_q8w_qkv_kv_dev(x, 8, wide, None, q, kv, 0, 0, pos)
        with pytest.raises(z.ZwgError, match="layer"):
            ctx.linear_q8w_qkv_kv_dev(x, 8, good, None, q, kv, 1, 0, pos)
        with pytest.raises(z.ZwgError, match="sequences"):
            ctx.linear_q8w_qkv_kv_dev(x, 8, good, None, q, kv, 0, 65, pos)
