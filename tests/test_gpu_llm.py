"""GPU parity of Qwen2's decode step on the device (zwg_llm_step_dev: Model.forward,
src/llm.zig:169-216, one token per sequence per step), and of the ops it adds, ops.rmsNorm and
ops.siluMul (zwg_rms_norm_dev, zwg_silu_mul_dev).

1. rms_norm_dev and silu_mul_dev against the oracle (f32 sums in other orders; the device's expf
   against the reference's expVec polynomial) and the f64 closed forms.
2. The step bit for bit against the same steps composed of the library's separate calls (RMS
   norm, the q/k/v projections writing the rotated cache, batched attention over the transposed
   cache, int8 linears with the add epilogue, the grouped gate/up call, SiLU-mul): logits and the
   caches equal over several steps, for head dims 32, 64 and 128 and GQA groups of 2 and 3, with a
   sequence whose position is off the cache and a token outside the vocabulary.  The embedding
   rows are checked against numpy's f32 embd.row.
3. Against the oracle (Oracle.llm_forward, the reference's forward one sequence at a time):
   logits within 2e-5 of the largest |logit| (measured 4e-7).
4. A step captured in a HIP graph and replayed equals the eager step; the shapes the call refuses.
5. The n-token forward (zwg_llm_forward_dev, the reference's prompt batch) against the oracle's
   forward over the same batches (40, 70 and 5 tokens), and against the same tokens one by one
   through the step; its refusals.
"""
from __future__ import annotations

import contextlib

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


def test_rms_norm_and_silu_mul(torch, ctx):
    import oracle

    rng = np.random.default_rng(1)
    with oracle.Oracle(2) as o:
        for m, n in ((7, 896), (3, 1536), (2, 4096 + 512), (5, 100)):
            x = (rng.standard_normal((m, n)) * rng.uniform(0.1, 30, (m, 1))).astype(np.float32)
            w = rng.standard_normal(n).astype(np.float32)
            out = torch.empty(m, n, device="cuda")
            ctx.rms_norm_dev(torch.from_numpy(x).cuda(), m, n, torch.from_numpy(w).cuda(), 1e-6, out)
            got = out.cpu().numpy()
            ref = o.rms_norm(x, m, n, w, 1e-6)
            x64 = x.astype(np.float64)
            f64 = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-6) * w
            scale = np.max(np.abs(f64))
            assert np.max(np.abs(got - ref)) <= 2e-6 * scale, (m, n)
            assert np.max(np.abs(got - f64)) <= 2e-6 * scale, (m, n)
        g = np.linspace(-30, 30, 4096).astype(np.float32)
        u = rng.standard_normal(4096).astype(np.float32)
        gt = torch.from_numpy(g).cuda()
        ctx.silu_mul_dev(gt, torch.from_numpy(u).cuda())
        got = gt.cpu().numpy()
        ref = o.silu_mul(g, u)
        f64 = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
        assert np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))) <= 2e-6
        assert np.max(np.abs(got - f64) / np.maximum(1.0, np.abs(f64))) <= 2e-6


def q8(rng, n, k):
    import zwhisper_amd as z

    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s = (rng.uniform(0.5, 1.5, (n, k // 32)) / 127 / np.sqrt(k) * 2).astype(np.float32)
    return z.Q8(q, s, n, k)


def model(rng, ne, H, Hk, nff, n_layer, n_vocab, tied=False):
    d = ne // H
    layers = []
    for _ in range(n_layer):
        layers.append({"wq": q8(rng, ne, ne), "wk": q8(rng, Hk * d, ne), "wv": q8(rng, Hk * d, ne),
                       "wo": q8(rng, ne, ne), "w_gate": q8(rng, nff, ne), "w_up": q8(rng, nff, ne),
                       "w_down": q8(rng, ne, nff),
                       "bq": (rng.standard_normal(ne) * 0.3).astype(np.float32),
                       "bk": (rng.standard_normal(Hk * d) * 0.3).astype(np.float32),
                       "bv": (rng.standard_normal(Hk * d) * 0.1).astype(np.float32),
                       "attn_norm": (1 + 0.1 * rng.standard_normal(ne)).astype(np.float32),
                       "ffn_norm": (1 + 0.1 * rng.standard_normal(ne)).astype(np.float32)})
    embd = q8(rng, n_vocab, ne)
    return {"embd": embd, "output": None if tied else q8(rng, n_vocab, ne),
            "output_norm": (1 + 0.1 * rng.standard_normal(ne)).astype(np.float32), "layers": layers}


def make_llm(z, ctx, mdl, H, Hk, nff, n_ctx, n_seq, base=1e6):
    return z.LLM(ctx, mdl["embd"], mdl["output"], mdl["output_norm"], mdl["layers"], H, Hk, nff, n_ctx, n_seq, base,
                 1e-6)


def embed_np(embd, tok):
    """embd.row(tok) in f32 (a zero row off the vocabulary)."""
    rows = np.zeros((len(tok), embd.k), np.float32)
    for i, t in enumerate(tok):
        if 0 <= t < embd.n:
            rows[i] = embd.row(int(t))
    return rows


def composed_step(torch, ctx, lm, kv, embd, H, Hk, tok, pos, seq0, logits):
    """The step as separate library calls over the fused model's own weights and its own cache."""
    import zwhisper_amd as z
    from zwhisper_amd import _lib

    ne, nff, m = lm.n_embd, lm.n_ff, len(tok)
    d = ne // H
    X = torch.empty(m, ne, device="cuda")
    Hn, Q, T = (torch.empty(m, ne, device="cuda") for _ in range(3))
    G, U = torch.empty(m, nff, device="cuda"), torch.empty(m, nff, device="cuda")
    X.copy_(torch.from_numpy(embed_np(embd, tok)))
    ctx.rms_norm_dev(X, m, ne, lm.layer_refs[0]["attn_norm"], lm.eps, Hn)
    pos_t = torch.from_numpy(np.asarray(pos, np.int32)).cuda()
    n_kv = torch.where((pos_t >= 0) & (pos_t < lm.n_ctx), pos_t + 1, torch.zeros_like(pos_t)).to(torch.int32)
    sh = z.AttnShape(1, lm.n_ctx, H, Hk, d, ne, Hk * d, ne, False, lm.n_ctx)
    for li, L in enumerate(lm.layer_refs):
        ctx.linear_q8w_qkv_kv_dev(Hn, m, [L["wq"], L["wk"], L["wv"]], [L["bq"], L["bk"], L["bv"]], Q, kv, li, seq0,
                                  pos_t)
        k, v = kv.ptrs(li, seq0)
        ps = kv.info.seq_stride
        ctx.attention_batch_dev(Q, k, v, sh, T, m, ne, ps, ps, ne, n_kv)
        ctx.linear_q8w_epi_dev(T, m, L["wo"], None, X, _lib.EPI_ADD)
        ctx.rms_norm_dev(X, m, ne, L["ffn_norm"], lm.eps, Hn)
        ctx.linear_q8w_group_dev(Hn, m, [L["w_gate"], L["w_up"]], None, [G, U])
        ctx.silu_mul_dev(G, U)
        ctx.linear_q8w_epi_dev(G, m, L["w_down"], None, X, _lib.EPI_ADD)
        nw = lm.output_norm if li + 1 == lm.n_layer else lm.layer_refs[li + 1]["attn_norm"]
        ctx.rms_norm_dev(X, m, ne, nw, lm.eps, Hn)
    ctx.linear_q8w_dev(Hn, m, lm.output, None, logits)


SHAPES = [(384, 6, 2, 1024), (512, 4, 2, 1376), (480, 15, 5, 864)]  # head dims 64, 128, 32


@pytest.mark.parametrize("ne,H,Hk,nff", SHAPES, ids=["d64", "d128", "d32"])
def test_step_bit_exact_with_composed_calls(torch, ctx, ne, H, Hk, nff):
    import zwhisper_amd as z
    from zwhisper_amd import _lib

    rng = np.random.default_rng(ne + H)
    n_layer, n_vocab, n_ctx, n_seq, seq0, m = 2, 700, 32, 8, 2, 5
    print(f"llm step n_embd={ne} heads {H}/{Hk} n_ff={nff} layers={n_layer} sequences {m} at {seq0}", flush=True)
    mdl = model(rng, ne, H, Hk, nff, n_layer, n_vocab, tied=(ne == 512))
    with contextlib.ExitStack() as st:
        lm = st.enter_context(make_llm(z, ctx, mdl, H, Hk, nff, n_ctx, n_seq))
        kv = st.enter_context(z.KVCache(ctx, n_layer, n_seq, n_ctx, Hk, ne // H, _lib.KV_KT, 1e6))
        start = np.array([0, 3, 7, 29, -1])
        la = torch.empty(m, n_vocab, device="cuda")
        lb = torch.empty(m, n_vocab, device="cuda")
        for step in range(3):
            pos = np.where(start >= 0, start + step, -1).astype(np.int32)
            tok = rng.integers(0, n_vocab, m).astype(np.int32)
            if step == 1:
                tok[2] = n_vocab + 3  # off the vocabulary: a zero embedding row
            lm.step(torch.from_numpy(tok).cuda(), torch.from_numpy(pos).cuda(), la, seq0)
            composed_step(torch, ctx, lm, kv, mdl["embd"], H, Hk, tok, pos, seq0, lb)
            torch.cuda.synchronize()
            assert torch.equal(la, lb), step
            assert torch.isfinite(la[torch.from_numpy(pos >= 0).cuda()]).all()
            for li in range(n_layer):
                for s in range(n_seq):
                    a, b = lm.kv.read(li, s), kv.read(li, s)
                    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), (step, li, s)


@pytest.mark.parametrize("m", [40, 64, 24])
def test_step_bit_exact_33_to_64_rows(torch, ctx, m):
    """33..64 sequences take the 64-row kernels, and (n_ff 8192 and a 16400-token vocabulary: the
    gate/up call and the logits stream a split x) the o projection's sum kernel splits the
    ffn-normed rows for the gate/up call and the last down projection's the output-normed rows
    for the logits, zero rows past m included.  At n_ff 8192 the SwiGLU pair is unsplit (its
    gate waves take the up waves' values); 24 sequences: the same with the 32-row kernels."""
    import zwhisper_amd as z
    from zwhisper_amd import _lib

    rng = np.random.default_rng(m)
    ne, H, Hk, nff, n_layer, n_vocab, n_ctx = 384, 6, 2, 8192, 2, 16400, 16
    print(f"llm step n_embd={ne} heads {H}/{Hk} n_ff={nff} layers={n_layer} sequences {m}", flush=True)
    mdl = model(rng, ne, H, Hk, nff, n_layer, n_vocab)
    with contextlib.ExitStack() as st:
        lm = st.enter_context(make_llm(z, ctx, mdl, H, Hk, nff, n_ctx, m))
        kv = st.enter_context(z.KVCache(ctx, n_layer, m, n_ctx, Hk, ne // H, _lib.KV_KT, 1e6))
        start = rng.integers(0, n_ctx - 2, m)
        start[3] = -1
        la = torch.empty(m, n_vocab, device="cuda")
        lb = torch.empty(m, n_vocab, device="cuda")
        for step in range(2):
            pos = np.where(start >= 0, start + step, -1).astype(np.int32)
            tok = rng.integers(0, n_vocab, m).astype(np.int32)
            lm.step(torch.from_numpy(tok).cuda(), torch.from_numpy(pos).cuda(), la, 0)
            composed_step(torch, ctx, lm, kv, mdl["embd"], H, Hk, tok, pos, 0, lb)
            torch.cuda.synchronize()
            assert torch.equal(la, lb), step
            for li in range(n_layer):
                for s in (0, 5, m - 1):
                    a, b = lm.kv.read(li, s), kv.read(li, s)
                    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), (step, li, s)


def test_step_against_oracle(torch, ctx):
    import oracle
    import zwhisper_amd as z
    from oracle import kv as kvo

    rng = np.random.default_rng(11)
    ne, H, Hk, nff, n_layer, n_vocab, n_ctx, m = 384, 6, 2, 1024, 2, 500, 32, 4
    d = ne // H
    print(f"llm step vs oracle n_embd={ne} heads {H}/{Hk} layers={n_layer} sequences {m}", flush=True)
    mdl = model(rng, ne, H, Hk, nff, n_layer, n_vocab)
    cos, sin = kvo.rope_tables(n_ctx, d, 1e6)
    ora_lm = {"embd": (mdl["embd"].q, mdl["embd"].scales), "output": (mdl["output"].q, mdl["output"].scales),
              "output_norm": mdl["output_norm"], "n_head": H, "n_head_kv": Hk, "eps": 1e-6, "cos": cos, "sin": sin,
              "layers": [{k: ((v.q, v.scales) if isinstance(v, z.Q8) else v) for k, v in lw.items()}
                         for lw in mdl["layers"]]}
    with contextlib.ExitStack() as st:
        o = st.enter_context(oracle.Oracle(4))
        lm = st.enter_context(make_llm(z, ctx, mdl, H, Hk, nff, n_ctx, m))
        caches = [{"kt": np.zeros((n_layer, Hk * d * n_ctx), np.float32), "v": np.zeros((n_layer, n_ctx, Hk * d),
                                                                                        np.float32)} for _ in range(m)]
        start = np.array([0, 2, 5, 11])
        logits = torch.empty(m, n_vocab, device="cuda")
        worst = 0.0
        for step in range(4):
            if step == 0:  # the sequences' earlier tokens, through both
                for w in range(m):
                    for p in range(start[w]):
                        t0 = int(rng.integers(0, n_vocab))
                        o.llm_forward(ora_lm, caches[w], t0, p)
                        tt = torch.zeros(m, dtype=torch.int32, device="cuda")
                        pp = torch.full((m,), -1, dtype=torch.int32, device="cuda")
                        tt[w], pp[w] = t0, p
                        lm.step(tt, pp, logits, 0)
            pos = (start + step).astype(np.int32)
            tok = rng.integers(0, n_vocab, m).astype(np.int32)
            lm.step(torch.from_numpy(tok).cuda(), torch.from_numpy(pos).cuda(), logits, 0)
            got = logits.cpu().numpy()
            for w in range(m):
                ref = o.llm_forward(ora_lm, caches[w], int(tok[w]), int(pos[w]))
                err = np.max(np.abs(got[w] - ref)) / max(1.0, np.max(np.abs(ref)))
                worst = max(worst, err)
                assert err <= 2e-5, (step, w, err)
        print(f"worst logit error {worst:.2e} of the largest |logit|", flush=True)


def _ora_model(z, mdl, H, Hk, n_ctx, d, base=1e6):
    from oracle import kv as kvo

    cos, sin = kvo.rope_tables(n_ctx, d, base)
    out = mdl["output"] if mdl["output"] is not None else mdl["embd"]
    return {"embd": (mdl["embd"].q, mdl["embd"].scales), "output": (out.q, out.scales),
            "output_norm": mdl["output_norm"], "n_head": H, "n_head_kv": Hk, "eps": 1e-6, "cos": cos, "sin": sin,
            "layers": [{k: ((v.q, v.scales) if isinstance(v, z.Q8) else v) for k, v in lw.items()}
                       for lw in mdl["layers"]]}


@pytest.mark.parametrize("ne,H,Hk,nff", [(384, 6, 2, 1024), (512, 4, 2, 1376)], ids=["d64", "d128"])
def test_forward_against_oracle(torch, ctx, ne, H, Hk, nff):
    """zwg_llm_forward_dev over prompt batches of 40, 70 (the tiled GEMMs past 64 rows) and 5
    tokens of sequence 1 against Oracle.llm_forward over the same batches: the last token's
    logits within 2e-5 of the largest |logit|, the cache rows within 2e-5 relative."""
    import oracle
    import zwhisper_amd as z

    rng = np.random.default_rng(ne + 1)
    n_layer, n_vocab, n_ctx, d = 2, 500, 128, ne // H
    print(f"llm forward vs oracle n_embd={ne} heads {H}/{Hk} n_ff={nff} layers={n_layer}", flush=True)
    mdl = model(rng, ne, H, Hk, nff, n_layer, n_vocab, tied=(ne == 512))
    ora = _ora_model(z, mdl, H, Hk, n_ctx, d)
    cache = {"kt": np.zeros((n_layer, Hk * d * n_ctx), np.float32), "v": np.zeros((n_layer, n_ctx, Hk * d), np.float32)}
    with contextlib.ExitStack() as st:
        o = st.enter_context(oracle.Oracle(4))
        lm = st.enter_context(make_llm(z, ctx, mdl, H, Hk, nff, n_ctx, 2))
        logits = torch.empty(n_vocab, device="cuda")
        pos = 0
        for n in (40, 70, 5):
            toks = rng.integers(0, n_vocab, n).astype(np.int32)
            lm.forward(torch.from_numpy(toks).cuda(), pos, logits, 1)
            ref = o.llm_forward(ora, cache, toks, pos)
            got = logits.cpu().numpy()
            scale = max(1.0, np.max(np.abs(ref)))
            err = np.max(np.abs(got - ref)) / scale
            print(f"  batch of {n} at {pos}: logit error {err:.2e} of the largest |logit|", flush=True)
            assert err <= 2e-5, (n, pos, err)
            pos += n
            for li in range(n_layer):
                k, v = lm.kv.read(li, 1)
                kr, vr = cache["kt"][li], cache["v"][li].reshape(-1)
                assert np.max(np.abs(k - kr)) <= 2e-5 * max(1.0, np.max(np.abs(kr))), li
                assert np.max(np.abs(v - vr)) <= 2e-5 * max(1.0, np.max(np.abs(vr))), li
                k0, _ = lm.kv.read(li, 0)
                assert not np.any(k0), "another sequence's cache was written"


def composed_forward(torch, ctx, lm, kv, embd, H, Hk, toks, pos0, seq, logits):
    """zwg_llm_forward_dev as separate library calls over the model's own weights and its own cache."""
    import zwhisper_amd as z
    from zwhisper_amd import _lib

    ne, nff, n = lm.n_embd, lm.n_ff, len(toks)
    d, kvw = ne // H, Hk * (ne // H)
    X, Hn, Q, T = (torch.empty(n, ne, device="cuda") for _ in range(4))
    Kb, Vb = torch.empty(n, kvw, device="cuda"), torch.empty(n, kvw, device="cuda")
    G, U = torch.empty(n, nff, device="cuda"), torch.empty(n, nff, device="cuda")
    X.copy_(torch.from_numpy(embed_np(embd, toks)))
    sh = z.AttnShape(n, pos0 + n, H, Hk, d, ne, kvw, ne, True, lm.n_ctx)
    for li, L in enumerate(lm.layer_refs):
        ctx.rms_norm_dev(X, n, ne, L["attn_norm"], lm.eps, Hn)
        ctx.linear_q8w_group_dev(Hn, n, [L["wq"], L["wk"], L["wv"]], [L["bq"], L["bk"], L["bv"]], [Q, Kb, Vb])
        kv.append(li, seq, pos0, Kb, Vb, Q, H, ne)
        k, v = kv.ptrs(li, seq)
        ctx.attention_dev(Q, k, v, sh, T)
        ctx.linear_q8w_epi_dev(T, n, L["wo"], None, X, _lib.EPI_ADD)
        ctx.rms_norm_dev(X, n, ne, L["ffn_norm"], lm.eps, Hn)
        ctx.linear_q8w_group_dev(Hn, n, [L["w_gate"], L["w_up"]], None, [G, U])
        ctx.silu_mul_dev(G, U)
        ctx.linear_q8w_epi_dev(G, n, L["w_down"], None, X, _lib.EPI_ADD)
    ctx.rms_norm_dev(X[n - 1:], 1, ne, lm.output_norm, lm.eps, Hn)
    ctx.linear_q8w_dev(Hn, 1, lm.output, None, logits)


@pytest.mark.parametrize("ne,H,Hk,nff", [(384, 6, 2, 1024), (480, 15, 5, 864), (384, 6, 2, 8192)],
                         ids=["d64", "d32", "ff8192"])
def test_forward_bit_exact_with_composed_calls(torch, ctx, ne, H, Hk, nff):
    """Prompt batches of at most 256 tokens (40, then 100: two 64-row blocks of the stream kernel,
    then 5) through the fused launches (the q/k/v projections writing the cache, the split sums
    adding into x and normalising it) equal the batch as separate calls bit for bit: the logits
    and the cache."""
    import zwhisper_amd as z
    from zwhisper_amd import _lib

    rng = np.random.default_rng(ne + nff)
    n_layer, n_vocab, n_ctx, seq = 2, 600, 160, 1
    mdl = model(rng, ne, H, Hk, nff, n_layer, n_vocab)
    with contextlib.ExitStack() as st:
        lm = st.enter_context(make_llm(z, ctx, mdl, H, Hk, nff, n_ctx, 2))
        kv = st.enter_context(z.KVCache(ctx, n_layer, 2, n_ctx, Hk, ne // H, _lib.KV_KT, 1e6))
        la = torch.empty(n_vocab, device="cuda")
        lb = torch.empty(n_vocab, device="cuda")
        pos = 0
        for n in (40, 100, 5):
            print(f"forward batch of {n} at {pos}", flush=True)
            toks = rng.integers(0, n_vocab, n).astype(np.int32)
            lm.forward(torch.from_numpy(toks).cuda(), pos, la, seq)
            composed_forward(torch, ctx, lm, kv, mdl["embd"], H, Hk, toks, pos, seq, lb)
            torch.cuda.synchronize()
            assert torch.equal(la, lb), n
            for li in range(n_layer):
                a, b = lm.kv.read(li, seq), kv.read(li, seq)
                assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), (n, li)
            pos += n


def test_forward_matches_steps(torch, ctx):
    """A prompt batch through zwg_llm_forward_dev and the same tokens one by one through
    zwg_llm_step_dev (other kernels): the last token's logits and the caches within f32
    rounding."""
    import zwhisper_amd as z

    rng = np.random.default_rng(77)
    ne, H, Hk, nff, n_layer, n_vocab, n_ctx = 384, 6, 2, 1024, 2, 400, 64
    mdl = model(rng, ne, H, Hk, nff, n_layer, n_vocab)
    toks = rng.integers(0, n_vocab, 33).astype(np.int32)
    with contextlib.ExitStack() as st:
        a = st.enter_context(make_llm(z, ctx, mdl, H, Hk, nff, n_ctx, 1))
        b = st.enter_context(make_llm(z, ctx, mdl, H, Hk, nff, n_ctx, 1))
        la = torch.empty(n_vocab, device="cuda")
        lb = torch.empty(1, n_vocab, device="cuda")
        a.forward(torch.from_numpy(toks).cuda(), 0, la, 0)
        for p, t in enumerate(toks):
            b.step(torch.tensor([t], dtype=torch.int32, device="cuda"), torch.tensor([p], dtype=torch.int32,
                                                                                      device="cuda"), lb, 0)
        torch.cuda.synchronize()
        ga, gb = la.cpu().numpy(), lb[0].cpu().numpy()
        assert np.max(np.abs(ga - gb)) <= 1e-5 * max(1.0, np.max(np.abs(gb)))
        for li in range(n_layer):
            ka, va = a.kv.read(li, 0)
            kb, vb = b.kv.read(li, 0)
            assert np.max(np.abs(ka - kb)) <= 1e-5 * max(1.0, np.max(np.abs(kb)))
            assert np.max(np.abs(va - vb)) <= 1e-5 * max(1.0, np.max(np.abs(vb)))


def test_forward_refusals(torch, ctx):
    import ctypes

    import zwhisper_amd as z
    from zwhisper_amd import _lib

    rng = np.random.default_rng(19)
    mdl = model(rng, 384, 6, 2, 256, 1, 64)
    L = _lib.lib()
    with make_llm(z, ctx, mdl, 6, 2, 256, 16, 2) as lm:
        logits = torch.empty(64, device="cuda")
        with pytest.raises(z.ZwgError, match="past the cache"):
            lm.forward(torch.zeros(10, dtype=torch.int32, device="cuda"), 7, logits, 0)
        with pytest.raises(z.ZwgError, match="sequences out of range"):
            lm.forward(torch.zeros(4, dtype=torch.int32, device="cuda"), 0, logits, 2)
        scratch = torch.empty(int(L.zwg_llm_forward_scratch(4, 384, 256)), device="cuda")
        rc = L.zwg_llm_forward_dev(ctx.handle, ctypes.byref(lm.c), None, 4, 0, 0, logits.data_ptr(),
                                   scratch.data_ptr())
        assert rc != 0 and "null tokens" in _lib.last_error(ctx.handle)


def test_step_graph_replay(torch, ctx):
    import zwhisper_amd as z

    rng = np.random.default_rng(5)
    ne, H, Hk, nff, n_vocab, m = 384, 6, 2, 1024, 300, 3
    mdl = model(rng, ne, H, Hk, nff, 2, n_vocab)
    with make_llm(z, ctx, mdl, H, Hk, nff, 32, m) as lm:
        tok = torch.from_numpy(rng.integers(0, n_vocab, m).astype(np.int32)).cuda()
        pos = torch.tensor([0, 4, 9], dtype=torch.int32, device="cuda")
        eager = torch.empty(m, n_vocab, device="cuda")
        lm.step(tok, pos, eager, 0)
        torch.cuda.synchronize()
        out = torch.empty(m, n_vocab, device="cuda")
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            lm.step(tok, pos, out, 0)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            lm.step(tok, pos, out, 0)
        for r in range(3):
            out.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), r
            lm.step(tok, pos, eager, 0)
            torch.cuda.synchronize()


def test_refusals(torch, ctx):
    import ctypes

    import zwhisper_amd as z
    from zwhisper_amd import _lib

    rng = np.random.default_rng(9)
    mdl = model(rng, 384, 6, 2, 256, 1, 64)
    L = _lib.lib()
    with make_llm(z, ctx, mdl, 6, 2, 256, 8, 2) as lm:
        tok = torch.zeros(65, dtype=torch.int32, device="cuda")
        logits = torch.empty(65, 64, device="cuda")
        with pytest.raises(z.ZwgError, match="at most 64"):
            lm.step(tok, tok, logits, 0)
        with pytest.raises(z.ZwgError, match="sequences out of range"):
            lm.step(tok[:2], tok[:2], logits, 1)

        def call(c):
            rc = L.zwg_llm_step_dev(ctx.handle, ctypes.byref(c), tok.data_ptr(), tok.data_ptr(), 1, 0,
                                    logits.data_ptr(), lm.scratch.data_ptr())
            return rc, _lib.last_error(ctx.handle)

        bad = _lib.LlmC.from_buffer_copy(lm.c)
        bad.n_head_kv = 4
        rc, msg = call(bad)
        assert rc != 0 and "n_head_kv" in msg
        bad = _lib.LlmC.from_buffer_copy(lm.c)
        bad.n_ff = 512
        rc, msg = call(bad)
        assert rc != 0 and "w_gate" in msg
        for layout, base in ((_lib.KV_ROW, 1e6), (_lib.KV_KT, 0.0)):
            with z.KVCache(ctx, 1, 2, 8, 2, 64, layout, base) as other:
                bad = _lib.LlmC.from_buffer_copy(lm.c)
                bad.kv = other._h.value
                rc, msg = call(bad)
                assert rc != 0 and "ZWG_KV_KT" in msg
