"""GPU parity of the Whisper decoder on the device (zwg_decoder_set_audio_dev, zwg_decoder_step_dev:
Decoder.setAudio and Decoder.forward, src/decoder.zig:151-205, one token per window per step).

1. Bit for bit against the same steps composed of the library's separate calls, each checked
   against f64 and the oracle elsewhere (layer norm, resident int8 linears with their epilogues,
   the q/k/v projections writing the cache, batched attention): logits, the self caches and the
   cross caches equal, over several steps, for head dims 32, 64 and 128, with a window whose
   position is off the cache and a token outside the vocabulary (the fused launches form the same
   values in the same order).  The embedding rows are checked against numpy's f32 te.row + pe.
2. Against the oracle (Oracle.decoder_set_audio / decoder_forward, the reference's forward one
   window at a time): logits within 2e-5 of the largest |logit| (f32 sums in other orders over two
   layers; measured 7e-7), cross caches within 1e-5 relative.
3. A step captured in a HIP graph and replayed, with eager work between the replays, equals the
   eager step; and the shapes the call refuses.
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


def q8(rng, n, k):
    import zwhisper_amd as z

    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s = (rng.uniform(0.5, 1.5, (n, k // 32)) / 127 / np.sqrt(k) * 2).astype(np.float32)
    return z.Q8(q, s, n, k)


def model(rng, ns, n_layer, n_vocab, n_ctx):
    def vec(n, scale=0.1):
        return (rng.standard_normal(n) * scale).astype(np.float32)

    layers = []
    for _ in range(n_layer):
        w = {}
        for name in ("q_w", "k_w", "v_w", "o_w", "cq_w", "ck_w", "cv_w", "co_w"):
            w[name] = q8(rng, ns, ns)
        w["mlp0_w"], w["mlp1_w"] = q8(rng, 4 * ns, ns), q8(rng, ns, 4 * ns)
        for name in ("q_b", "v_b", "o_b", "cq_b", "cv_b", "co_b", "mlp1_b"):
            w[name] = vec(ns)
        w["mlp0_b"] = vec(4 * ns)
        for ln in ("attn_ln", "cross_ln", "mlp_ln"):
            w[ln + "_w"], w[ln + "_b"] = 1 + vec(ns), vec(ns)
        layers.append(w)
    return dict(te=q8(rng, n_vocab, ns), pe=(rng.standard_normal((n_ctx, ns)) * 0.5).astype(np.float32),
                ln_w=1 + vec(ns), ln_b=vec(ns), layers=layers)


def embed_np(te, pe, tok, pos):
    """te.row(tok) + pe[pos] in f32 (zero row off the vocabulary, no position row off the cache)."""
    ns = te.k
    rows = np.zeros((len(tok), ns), np.float32)
    for i, (t, p) in enumerate(zip(tok, pos)):
        if 0 <= t < te.n:
            rows[i] = te.row(int(t))
        if 0 <= p < pe.shape[0]:
            rows[i] = rows[i] + pe[p]
    return rows


class Composed:
    """The decoder step as separate library calls over the fused decoder's own weights."""

    def __init__(self, torch, ctx, dec, n_head, n_windows):
        import zwhisper_amd as z

        self.t, self.ctx, self.dec, self.H = torch, ctx, dec, n_head
        ns = dec.n_state
        d = ns // n_head
        self.self_kv = z.KVCache(ctx, dec.n_layer, n_windows, dec.n_text_ctx, n_head, d)
        self.cross_kv = z.KVCache(ctx, dec.n_layer, n_windows, dec.n_audio_ctx, n_head, d)
        self.X, self.A, self.Q, self.T = (torch.empty(64, ns, device="cuda") for _ in range(4))
        self.Hd = torch.empty(64, 4 * ns, device="cuda")

    def close(self):
        self.self_kv.close()
        self.cross_kv.close()

    def set_audio(self, enc, n_windows, seq0):
        rows = n_windows * self.dec.n_audio_ctx
        for li, L in enumerate(self.dec.layer_refs):
            k, v = self.cross_kv.ptrs(li, seq0)
            self.ctx.linear_q8w_dev(enc, rows, L["ck_w"], None, k)
            self.ctx.linear_q8w_dev(enc, rows, L["cv_w"], L["cv_b"], v)

    def step(self, te_host, pe_host, tok, pos, seq0, logits):
        import zwhisper_amd as z
        from zwhisper_amd import _lib

        t, ctx, dec = self.t, self.ctx, self.dec
        ns, m = dec.n_state, len(tok)
        X, A, Q, T, Hd = self.X, self.A, self.Q, self.T, self.Hd
        X[:m] = t.from_numpy(embed_np(te_host, pe_host, tok, pos)).cuda()
        L0 = dec.layer_refs[0]
        ctx.layer_norm_dev(X, m, ns, L0["attn_ln_w"], L0["attn_ln_b"], 1e-5, A)
        pos_t = t.from_numpy(np.asarray(pos, np.int32)).cuda()
        n_kv = t.where((pos_t >= 0) & (pos_t < dec.n_text_ctx), pos_t + 1, t.zeros_like(pos_t)).to(t.int32)
        sh_self = z.AttnShape(1, dec.n_text_ctx, self.H, self.H, ns // self.H, ns, ns, ns, False)
        sh_cross = z.AttnShape(1, dec.n_audio_ctx, self.H, self.H, ns // self.H, ns, ns, ns, False)
        for li, L in enumerate(dec.layer_refs):
            ctx.linear_q8w_qkv_kv_dev(A, m, [L["q_w"], L["k_w"], L["v_w"]], [L["q_b"], None, L["v_b"]], Q,
                                      self.self_kv, li, seq0, pos_t)
            k, v = self.self_kv.ptrs(li, seq0)
            ps = self.self_kv.info.seq_stride
            ctx.attention_batch_dev(Q, k, v, sh_self, T, m, ns, ps, ps, ns, n_kv)
            ctx.linear_q8w_epi_dev(T, m, L["o_w"], L["o_b"], X, _lib.EPI_ADD)
            ctx.layer_norm_dev(X, m, ns, L["cross_ln_w"], L["cross_ln_b"], 1e-5, A)
            ctx.linear_q8w_dev(A, m, L["cq_w"], L["cq_b"], Q)
            k, v = self.cross_kv.ptrs(li, seq0)
            pc = self.cross_kv.info.seq_stride
            ctx.attention_batch_dev(Q, k, v, sh_cross, T, m, ns, pc, pc, ns)
            ctx.linear_q8w_epi_dev(T, m, L["co_w"], L["co_b"], X, _lib.EPI_ADD)
            ctx.layer_norm_dev(X, m, ns, L["mlp_ln_w"], L["mlp_ln_b"], 1e-5, A)
            ctx.linear_q8w_epi_dev(A, m, L["mlp0_w"], L["mlp0_b"], Hd, _lib.EPI_GELU)
            ctx.linear_q8w_epi_dev(Hd, m, L["mlp1_w"], L["mlp1_b"], X, _lib.EPI_ADD)
            last = li + 1 == dec.n_layer
            nw = dec.ln_w if last else dec.layer_refs[li + 1]["attn_ln_w"]
            nb = dec.ln_b if last else dec.layer_refs[li + 1]["attn_ln_b"]
            ctx.layer_norm_dev(X, m, ns, nw, nb, 1e-5, A)
        ctx.linear_q8w_dev(A, m, dec.te, None, logits)


def make_decoder(z, ctx, mdl, n_head, n_text_ctx, n_audio_ctx, n_windows):
    return z.Decoder(ctx, mdl["te"], mdl["pe"], mdl["ln_w"], mdl["ln_b"], mdl["layers"], n_head, n_text_ctx,
                     n_audio_ctx, n_windows)


SHAPES = [(384, 6), (512, 4), (320, 10)]  # head dims 64, 128, 32


@pytest.mark.parametrize("ns,H", SHAPES, ids=["d64", "d128", "d32"])
def test_step_bit_exact_with_composed_calls(torch, ctx, ns, H):
    import zwhisper_amd as z

    rng = np.random.default_rng(ns + H)
    n_layer, n_vocab, n_tctx, n_actx, n_win, seq0, m = 2, 700, 24, 100, 8, 2, 5
    print(f"decoder step n_state={ns} heads={H} layers={n_layer} windows {m} at {seq0}", flush=True)
    mdl = model(rng, ns, n_layer, n_vocab, n_tctx)
    with contextlib.ExitStack() as st:
        dec = st.enter_context(make_decoder(z, ctx, mdl, H, n_tctx, n_actx, n_win))
        comp = Composed(torch, ctx, dec, H, n_win)
        st.callback(comp.close)
        enc = torch.from_numpy(rng.standard_normal((m, n_actx, ns)).astype(np.float32)).cuda()
        dec.set_audio(enc, m, seq0)
        comp.set_audio(enc, m, seq0)
        torch.cuda.synchronize()
        for li in range(n_layer):
            for s in range(n_win):
                a, b = dec.cross_kv.read(li, s), comp.cross_kv.read(li, s)
                assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), (li, s)
        start = np.array([0, 3, 7, 21, -1])
        la = torch.empty(m, n_vocab, device="cuda")
        lb = torch.empty(m, n_vocab, device="cuda")
        for step in range(3):
            pos = np.where(start >= 0, start + step, -1).astype(np.int32)
            tok = rng.integers(0, n_vocab, m).astype(np.int32)
            tok[2] = n_vocab + 3 if step == 1 else tok[2]  # off the vocabulary: a zero embedding row
            dec.step(torch.from_numpy(tok).cuda(), torch.from_numpy(pos).cuda(), la, seq0)
            comp.step(mdl["te"], mdl["pe"], tok, pos, seq0, lb)
            torch.cuda.synchronize()
            assert torch.equal(la, lb), step
            assert torch.isfinite(la[pos >= 0]).all()
            for li in range(n_layer):
                for s in range(n_win):
                    a, b = dec.self_kv.read(li, s), comp.self_kv.read(li, s)
                    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), (step, li, s)


def test_step_against_oracle(torch, ctx):
    import oracle
    import zwhisper_amd as z

    rng = np.random.default_rng(21)
    ns, H, n_layer, n_vocab, n_tctx, n_actx, m = 384, 6, 2, 500, 16, 100, 4
    print(f"decoder step vs oracle n_state={ns} heads={H} layers={n_layer} windows {m}", flush=True)
    mdl = model(rng, ns, n_layer, n_vocab, n_tctx)
    ora_layers = [{k: ((v.q, v.scales) if isinstance(v, z.Q8) else v) for k, v in lw.items()} for lw in mdl["layers"]]
    ora_dec = {"te": (mdl["te"].q, mdl["te"].scales), "pe": mdl["pe"], "ln_w": mdl["ln_w"], "ln_b": mdl["ln_b"],
               "n_head": H, "layers": ora_layers}
    with contextlib.ExitStack() as st:
        o = st.enter_context(oracle.Oracle(4))
        dec = st.enter_context(make_decoder(z, ctx, mdl, H, n_tctx, n_actx, m))
        enc = rng.standard_normal((m, n_actx, ns)).astype(np.float32)
        dec.set_audio(torch.from_numpy(enc).cuda(), m, 0)
        caches = []
        for w in range(m):
            cross = o.decoder_set_audio(enc[w], n_actx, ns, ora_layers)
            for li, (ck, cv) in enumerate(cross):
                gk, gv = dec.cross_kv.read(li, w)
                for g, r in ((gk, ck), (gv, cv)):
                    assert np.max(np.abs(g.reshape(r.shape) - r)) <= 1e-5 * max(1.0, np.max(np.abs(r)))
            caches.append({"k": np.zeros((n_layer, n_tctx, ns), np.float32),
                           "v": np.zeros((n_layer, n_tctx, ns), np.float32),
                           "ck": np.stack([c[0] for c in cross]), "cv": np.stack([c[1] for c in cross])})
        start = np.array([0, 2, 5, 11])
        logits = torch.empty(m, n_vocab, device="cuda")
        worst = 0.0
        for step in range(4):
            pos = (start + step).astype(np.int32)
            tok = rng.integers(0, n_vocab, m).astype(np.int32)
            if step == 0:  # the windows' earlier tokens, through both
                for w in range(m):
                    for p in range(start[w]):
                        t0 = int(rng.integers(0, n_vocab))
                        o.decoder_forward(ora_dec, caches[w], t0, p)
                        tt = torch.full((m,), 0, dtype=torch.int32, device="cuda")
                        pp = torch.full((m,), -1, dtype=torch.int32, device="cuda")
                        tt[w], pp[w] = t0, p
                        dec.step(tt, pp, logits, 0)
            dec.step(torch.from_numpy(tok).cuda(), torch.from_numpy(pos).cuda(), logits, 0)
            got = logits.cpu().numpy()
            for w in range(m):
                ref = o.decoder_forward(ora_dec, caches[w], int(tok[w]), int(pos[w]))
                err = np.max(np.abs(got[w] - ref)) / max(1.0, np.max(np.abs(ref)))
                worst = max(worst, err)
                assert err <= 2e-5, (step, w, err)
        print(f"worst logit error {worst:.2e} of the largest |logit|", flush=True)


def test_step_graph_replay(torch, ctx):
    import zwhisper_amd as z

    rng = np.random.default_rng(5)
    ns, H, n_layer, n_vocab, n_tctx, n_actx, m = 384, 6, 2, 300, 16, 64, 3
    mdl = model(rng, ns, n_layer, n_vocab, n_tctx)
    with make_decoder(z, ctx, mdl, H, n_tctx, n_actx, m) as dec:
        dec.set_audio(torch.from_numpy(rng.standard_normal((m, n_actx, ns)).astype(np.float32)).cuda(), m, 0)
        tok = torch.from_numpy(rng.integers(0, n_vocab, m).astype(np.int32)).cuda()
        pos = torch.tensor([0, 4, 9], dtype=torch.int32, device="cuda")
        eager = torch.empty(m, n_vocab, device="cuda")
        dec.step(tok, pos, eager, 0)
        torch.cuda.synchronize()
        out = torch.empty(m, n_vocab, device="cuda")
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            dec.step(tok, pos, out, 0)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            dec.step(tok, pos, out, 0)
        for r in range(3):
            out.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), r
            dec.step(tok, pos, eager, 0)  # eager work between replays
            torch.cuda.synchronize()


def test_refusals(torch, ctx):
    import ctypes

    import zwhisper_amd as z
    from zwhisper_amd import _lib

    rng = np.random.default_rng(9)
    mdl = model(rng, 384, 1, 64, 8)
    with make_decoder(z, ctx, mdl, 6, 8, 32, 2) as dec:
        tok = torch.zeros(65, dtype=torch.int32, device="cuda")
        logits = torch.empty(65, 64, device="cuda")
        with pytest.raises(z.ZwgError, match="at most 64"):
            dec.step(tok, tok, logits, 0)
        with pytest.raises(z.ZwgError, match="windows out of range"):
            dec.step(tok[:2], tok[:2], logits, 1)
        bad = _lib.DecoderC.from_buffer_copy(dec.c)
        bad.n_head = 5
        L = _lib.lib()
        rc = L.zwg_decoder_step_dev(ctx.handle, ctypes.byref(bad), tok.data_ptr(), tok.data_ptr(), 1, 0,
                                    logits.data_ptr(), dec.scratch.data_ptr())
        assert rc != 0 and "multiple of n_head" in _lib.last_error(ctx.handle)
        bad = _lib.DecoderC.from_buffer_copy(dec.c)
        bad.n_vocab = 65
        rc = L.zwg_decoder_step_dev(ctx.handle, ctypes.byref(bad), tok.data_ptr(), tok.data_ptr(), 1, 0,
                                    logits.data_ptr(), dec.scratch.data_ptr())
        assert rc != 0 and "te" in _lib.last_error(ctx.handle)
        with z.KVCache(ctx, 1, 2, 8, 6, 64, _lib.KV_ROW, 1e4) as rope:
            bad = _lib.DecoderC.from_buffer_copy(dec.c)
            bad.self_kv = rope._h.value
            rc = L.zwg_decoder_step_dev(ctx.handle, ctypes.byref(bad), tok.data_ptr(), tok.data_ptr(), 1, 0,
                                        logits.data_ptr(), dec.scratch.data_ptr())
            assert rc != 0 and "no rotary" in _lib.last_error(ctx.handle)
    small = model(rng, 256, 1, 64, 8)
    with pytest.raises(z.ZwgError, match="above 256"):
        with make_decoder(z, ctx, small, 4, 8, 32, 2) as dec:
            dec.step(tok[:1], tok[:1], logits, 0)
