"""GPU parity of the device-resident KV caches (zwg_kv_*) against oracle/kv.py.

Cache contents must match the oracle bit for bit: appends are copies, and the rotary
positions are computed from identical f32 tables with every product and sum rounded as the
reference rounds them.  Attention read straight from the device caches is then checked against
the oracle's attention over the oracle's caches, to the f32 bar (max abs 2e-4, normwise rel
1e-3).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import kv as okv
from zwhisper_amd import _lib
from zwhisper_amd.ops import AttnShape

pytestmark = pytest.mark.gpu

BASE = 1.0e6


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


def rng_f32(seed, *shape):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def test_row_cache_appends_bit_exact(torch, ctx):
    """Whisper decoder caches [n_ctx][n_state]: prompt rows, then tokens one at a time
    (src/decoder.zig:182-183), in two layers and two windows."""
    import zwhisper_amd as z

    n_ctx, h, d = 448, 12, 64
    kvw = h * d
    with z.KVCache(ctx, 2, 2, n_ctx, h, d, z.KV_ROW) as kv:
        ref = {(l, s): (np.zeros(n_ctx * kvw, np.float32), np.zeros(n_ctx * kvw, np.float32)) for l in range(2) for s in range(2)}
        seed = 10
        for l, s, pos, n in [(0, 0, 0, 4), (0, 0, 4, 1), (0, 0, 5, 1), (1, 1, 0, 33), (1, 1, 33, 1), (0, 1, 0, 448),
                             (1, 0, 447, 1)]:
            k, v = rng_f32(seed, n, kvw), rng_f32(seed + 1, n, kvw)
            seed += 2
            kv.append(l, s, pos, dev(torch, k), dev(torch, v))
            okv.append_rows(ref[(l, s)][0], kvw, pos, k, n)
            okv.append_rows(ref[(l, s)][1], kvw, pos, v, n)
        torch.cuda.synchronize()
        for key, (rk, rv) in ref.items():
            gk, gv = kv.read(*key)
            assert np.array_equal(gk, rk) and np.array_equal(gv, rv), key


@pytest.mark.parametrize("d,hkv,h", [(128, 2, 12), (64, 2, 14)])
def test_kt_cache_rope_bit_exact(torch, ctx, d, hkv, h):
    """Qwen2 caches: rotary positions on k and q, transposed scatter, v rows (src/llm.zig:182-190),
    for a prompt in batches and then single tokens."""
    import zwhisper_amd as z

    n_ctx = 1024
    kvw, ne = hkv * d, h * d
    cos, sin = okv.rope_tables(n_ctx, d, BASE)
    with z.KVCache(ctx, 1, 1, n_ctx, hkv, d, z.KV_KT, rope_base=BASE) as kv:
        rkt = np.zeros(hkv * d * n_ctx, np.float32)
        rv = np.zeros(n_ctx * kvw, np.float32)
        n_past, seed = 0, 100
        for n in (256, 256, 100, 1, 1, 17, 1):
            q, k, v = rng_f32(seed, n, ne), rng_f32(seed + 1, n, kvw), rng_f32(seed + 2, n, kvw)
            seed += 3
            qd = dev(torch, q)
            kv.append(0, 0, n_past, dev(torch, k), dev(torch, v), qd, h, ne)
            okv.llm_append(q, k, v, n, n_past, h, hkv, d, ne, rkt, rv, n_ctx, cos, sin)
            torch.cuda.synchronize()
            assert np.array_equal(qd.cpu().numpy(), q), f"q rotation at n_past={n_past}"
            n_past += n
        gk, gv = kv.read(0, 0)
        assert np.array_equal(gk, rkt)
        assert np.array_equal(gv, rv)


def test_host_rows_path(torch, ctx):
    """ZWG_ROWS_ON_HOST: the same cache and the same rotated q from host buffers."""
    import zwhisper_amd as z

    n_ctx, hkv, h, d = 256, 2, 12, 128
    kvw, ne = hkv * d, h * d
    cos, sin = okv.rope_tables(n_ctx, d, BASE)
    q, k, v = rng_f32(200, 5, ne), rng_f32(201, 5, kvw), rng_f32(202, 5, kvw)
    with z.KVCache(ctx, 1, 1, n_ctx, hkv, d, z.KV_KT, rope_base=BASE) as kv:
        qh = q.copy()
        kv.append(0, 0, 7, k, v, qh, h, ne)
        rkt = np.zeros(hkv * d * n_ctx, np.float32)
        rv = np.zeros(n_ctx * kvw, np.float32)
        qr = q.copy()
        okv.llm_append(qr, k, v, 5, 7, h, hkv, d, ne, rkt, rv, n_ctx, cos, sin)
        gk, gv = kv.read(0, 0)
        assert np.array_equal(gk, rkt) and np.array_equal(gv, rv)
        assert np.array_equal(qh, qr)


def test_batch_append_per_sequence_positions(torch, ctx):
    """One token for each of 64 sequences at its own position (a batched decode step); a position
    outside [0, n_ctx) is skipped."""
    import zwhisper_amd as z

    n_seq, n_ctx, hkv, h, d = 64, 4096, 2, 12, 128
    kvw, ne = hkv * d, h * d
    cos, sin = okv.rope_tables(n_ctx, d, BASE)
    pos = np.random.default_rng(300).integers(0, n_ctx, n_seq).astype(np.int32)
    pos[5] = n_ctx  # out of range: skipped
    pos[9] = -1
    q, k, v = rng_f32(301, n_seq, ne), rng_f32(302, n_seq, kvw), rng_f32(303, n_seq, kvw)
    with z.KVCache(ctx, 2, n_seq, n_ctx, hkv, d, z.KV_KT, rope_base=BASE) as kv:
        qd = dev(torch, q)
        kv.append_batch(1, 0, torch.from_numpy(pos).cuda(), dev(torch, k), dev(torch, v), qd, h, ne)
        torch.cuda.synchronize()
        gq = qd.cpu().numpy()
        for s in range(n_seq):
            rkt = np.zeros(hkv * d * n_ctx, np.float32)
            rv = np.zeros(n_ctx * kvw, np.float32)
            qs = q[s:s + 1].copy()
            if 0 <= pos[s] < n_ctx:
                okv.llm_append(qs, k[s:s + 1], v[s:s + 1], 1, int(pos[s]), h, hkv, d, ne, rkt, rv, n_ctx, cos, sin)
            gk, gv = kv.read(1, s)
            assert np.array_equal(gk, rkt) and np.array_equal(gv, rv), s
            assert np.array_equal(gq[s], qs[0]), s
        gk, gv = kv.read(0, 3)  # the other layer untouched
        assert not gk.any() and not gv.any()


def test_decoder_attention_reads_device_cache(torch, ctx):
    """A Whisper decoder self-attention step over caches filled on the device, for 8 windows of
    different lengths, read in place by one batched attention call."""
    import zwhisper_amd as z

    n_win, n_ctx, h, d = 8, 448, 12, 64
    ns = h * d
    lengths = np.array([1, 2, 17, 100, 255, 256, 300, 448], np.int32)
    o = oracle.Oracle(2)
    with z.KVCache(ctx, 1, n_win, n_ctx, h, d, z.KV_ROW) as kv:
        caches = []
        for w in range(n_win):
            k, v = rng_f32(400 + w, int(lengths[w]), ns), rng_f32(500 + w, int(lengths[w]), ns)
            kv.append(0, w, 0, dev(torch, k), dev(torch, v))
            caches.append((k, v))
        q = rng_f32(600, n_win, ns)
        out = torch.zeros(n_win * ns, device="cuda")
        kp, vp = kv.ptrs(0, 0)
        sh = AttnShape(1, n_ctx, h, h, d, ns, ns, ns, True, None)
        ctx.attention_batch_dev(dev(torch, q), kp, vp, sh, out, n_win, ns, kv.info.seq_stride, kv.info.seq_stride, ns,
                                torch.from_numpy(lengths).cuda())
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(n_win, ns)
        for w in range(n_win):
            k, v = caches[w]
            ref = o.attention_ex(q[w], k.reshape(-1), v.reshape(-1),
                                 AttnShape(1, int(lengths[w]), h, h, d, ns, ns, ns, True, None))
            err = float(np.abs(got[w] - ref).max())
            assert err <= 2e-4, (w, err)
    o.close()


def test_llm_decode_reads_device_cache(torch, ctx):
    """Qwen2-1.5B-shaped decode (12/2 heads x 128): a prompt appended with rotary positions, then
    one more token per sequence through the batch append, then attention over the transposed
    device caches -- against the oracle's attention over the oracle's caches."""
    import zwhisper_amd as z

    n_seq, n_ctx, hkv, h, d = 4, 512, 2, 12, 128
    kvw, ne = hkv * d, h * d
    cos, sin = okv.rope_tables(n_ctx, d, BASE)
    prompt = [37, 300, 1, 128]
    o = oracle.Oracle(2)
    with z.KVCache(ctx, 1, n_seq, n_ctx, hkv, d, z.KV_KT, rope_base=BASE) as kv:
        refs = []
        for s in range(n_seq):
            n = prompt[s]
            k, v = rng_f32(700 + s, n, kvw), rng_f32(710 + s, n, kvw)
            kv.append(0, s, 0, dev(torch, k), dev(torch, v))
            rkt = np.zeros(hkv * d * n_ctx, np.float32)
            rv = np.zeros(n_ctx * kvw, np.float32)
            okv.llm_append(None, k, v, n, 0, h, hkv, d, ne, rkt, rv, n_ctx, cos, sin)
            refs.append((rkt, rv))
        pos = np.array(prompt, np.int32)
        q, k, v = rng_f32(720, n_seq, ne), rng_f32(721, n_seq, kvw), rng_f32(722, n_seq, kvw)
        qd = dev(torch, q)
        kv.append_batch(0, 0, torch.from_numpy(pos).cuda(), dev(torch, k), dev(torch, v), qd, h, ne)
        n_kv = pos + 1
        out = torch.zeros(n_seq * ne, device="cuda")
        kp, vp = kv.ptrs(0, 0)
        sh = AttnShape(1, n_ctx, h, hkv, d, ne, kvw, ne, True, n_ctx)
        ctx.attention_batch_dev(qd, kp, vp, sh, out, n_seq, ne, kv.info.seq_stride, kv.info.seq_stride, ne,
                                torch.from_numpy(n_kv.astype(np.int32)).cuda())
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(n_seq, ne)
        for s in range(n_seq):
            rkt, rv = refs[s]
            qs = q[s:s + 1].copy()
            okv.llm_append(qs, k[s:s + 1], v[s:s + 1], 1, int(pos[s]), h, hkv, d, ne, rkt, rv, n_ctx, cos, sin)
            ref = o.attention_ex(qs.reshape(-1), rkt, rv, AttnShape(1, int(n_kv[s]), h, hkv, d, ne, kvw, ne, True, n_ctx))
            err = float(np.abs(got[s] - ref).max())
            assert err <= 2e-4, (s, err)
    o.close()


def test_kv_errors(torch, ctx):
    import zwhisper_amd as z

    with pytest.raises(z.ZwgError, match="multiple of 4"):
        z.KVCache(ctx, 1, 1, 30, 2, 64, z.KV_KT)
    with pytest.raises(z.ZwgError, match="head dim"):
        z.KVCache(ctx, 1, 1, 32, 2, 48, z.KV_ROW)
    with z.KVCache(ctx, 1, 1, 16, 2, 64, z.KV_ROW) as kv:
        rows = torch.zeros(4 * 128, device="cuda")
        with pytest.raises(z.ZwgError, match="past the end"):
            kv.append(0, 0, 14, rows, rows)
        with pytest.raises(z.ZwgError, match="rope_base"):
            kv.append(0, 0, 0, rows, rows, torch.zeros(4 * 128, device="cuda"), 2, 128)
        with pytest.raises(z.ZwgError, match="layer"):
            kv.append(1, 0, 0, rows, rows)
        assert _lib.last_error(ctx.handle)
