"""An independent float64 Whisper, written from the published architecture
(Radford et al. 2022, "Robust Speech Recognition via Large-Scale Weak
Supervision", and the layer list of the ggml model format), NOT from the
oracle's C source.  It is the check that pins how the oracle composes its
primitives: conv stem, positional embedding, pre-LN blocks, which linears carry
a bias, the attention scale, the causal mask, cross-attention over the encoder
states, ln_post, the tied logits head and the greedy loop.

Arithmetic is float64 throughout.  Three reference numerics are part of the
model definition rather than of its arithmetic order, so they are options:

  gelu="f16"    the reference GELU is a lookup of the f16-rounded input in a
                table of f16-rounded tanh-GELU values, identity at x >= 10 and
                zero at x <= -10 (nn.rs:4561-4687); gelu="exact" is the plain
                tanh-approximation GELU in float64.
  kv_f16=True   the decoder's self-attention cache stores K and V rounded to
                f16 (FW_KV_F16, nn.rs:5352-5416).
  cross_f16=True the cross-attention keys and values are held as f16
                (decoder.rs:1154-1222).

`mutate` plants one named mistake, so a test can show that the comparison
against the oracle would catch it (see MUTATIONS).

TEST INFRASTRUCTURE: used only by tests/.
"""
from __future__ import annotations

import numpy as np

MUTATIONS = (
    "no_q_bias",          # drop the query bias (encoder and decoder)
    "no_v_bias",          # drop the value bias
    "no_o_bias",          # drop the attention output bias
    "no_fc1_bias",
    "no_fc2_bias",
    "k_bias_from_q",      # give the key projection the query's bias
    "attn_unscaled",      # no 1/sqrt(d_head) on the scores
    "attn_scale_full_k",  # d_head^-0.5 on K and on q (scale applied twice)
    "conv_taps_reversed",  # conv kernel taps in the opposite order
    "conv2_stride1_even",  # stride-2 conv takes odd instead of even centres
    "no_pos_emb",         # skip the positional embedding
    "no_ln_post",         # skip the encoder's final LayerNorm
    "no_causal_mask",     # decoder self-attention sees future prompt rows
    "cross_k_unscaled",   # cross-attention scores without the scale
    "no_cross_v_bias",    # cross V projection without its bias
    "no_final_ln",        # decoder's final LayerNorm skipped
    "pos_emb_shift",      # decoder positional embedding off by one
    "ln_eps_1e-3",        # LayerNorm epsilon 1e-3 instead of 1e-5
    "gelu_erf",           # erf GELU instead of the tanh approximation
    "tome_no_average",    # ToMe adds merged rows into their partner without dividing by the count
    "tome_merge_lowest",  # ToMe merges the r least similar A rows instead of the most similar
    "tome_dot_not_cos",   # ToMe ranks by the raw dot product instead of the cosine
    "tome_every_off_by_one",  # the progressive schedule merges one block after each due block
    "tome_ignore_floor",  # the progressive schedule merges past the floor
)


def f16(a):
    """Round float64 values to the nearest f16 (RNE) and back."""
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float64)


def w16(u16):
    """ggml f16 tensor (raw uint16 bits) -> float64."""
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float64)


class Numerics:
    def __init__(self, gelu="f16", kv_f16=True, cross_f16=True, mutate=None):
        assert gelu in ("f16", "exact")
        assert mutate is None or mutate in MUTATIONS, mutate
        self.gelu_mode, self.kv_f16, self.cross_f16, self.mutate = gelu, kv_f16, cross_f16, mutate

    def m(self, name):
        return self.mutate == name

    def gelu(self, x):
        x = np.asarray(x, np.float64)
        if self.m("gelu_erf"):
            from scipy.special import erf
            return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))

        def g(v):
            return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))
        if self.gelu_mode == "exact":
            return g(x)
        y = f16(g(f16(x)))
        return np.where(x <= -10.0, 0.0, np.where(x >= 10.0, x, y))

    def ln(self, x, w, b):
        eps = 1e-3 if self.m("ln_eps_1e-3") else 1e-5
        mu = x.mean(axis=-1, keepdims=True)
        var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
        return (x - mu) / np.sqrt(var + eps) * w + b


def softmax(s):
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return e / e.sum(axis=-1, keepdims=True)


def mha(q, k, v, n_head, nm: Numerics, causal_offset=None, kv_round=None):
    """Multi-head attention on [tq, d] x [tk, d]; causal_offset=c lets query i
    see keys j <= c + i."""
    tq, d = q.shape
    tk = k.shape[0]
    dh = d // n_head
    if nm.m("attn_unscaled"):
        scale = 1.0
    elif nm.m("attn_scale_full_k"):
        scale = 1.0 / dh
    else:
        scale = 1.0 / np.sqrt(dh)
    out = np.empty((tq, d))
    for h in range(n_head):
        sl = slice(h * dh, (h + 1) * dh)
        s = (q[:, sl] @ k[:, sl].T) * scale
        if causal_offset is not None and not nm.m("no_causal_mask"):
            j = np.arange(tk)[None, :]
            i = np.arange(tq)[:, None]
            s = np.where(j > causal_offset + i, -np.inf, s)
        out[:, sl] = softmax(s) @ v[:, sl]
    return out


def tome_merge(x, r, nm: Numerics | None = None):
    """Token merging by bipartite soft matching (Bolya et al. 2023, "Token
    Merging: Your ViT but Faster"), single shot: even rows form set A, odd rows
    set B; each A row's edge goes to its most cosine-similar B row (the first
    one on a tie); the r A rows with the most similar edges are averaged into
    their B partners (a B row's result is the mean of itself and every A row
    merged into it); the merged sequence is the B rows followed by the kept A
    rows in their order.  Returns the merged rows, the map from each original
    row to its merged row, and the decision margins (how far the r-th best edge
    is from the next, and the smallest best-vs-second-best gap of a merged row)
    so a caller can check that float32 and float64 must agree on the decisions."""
    nm = nm or Numerics()
    x = np.asarray(x, np.float64)
    seq = x.shape[0]
    A, B = x[0::2], x[1::2]
    n_a, n_b = A.shape[0], B.shape[0]
    r = min(r, n_a, seq - 1)
    sim = A @ B.T
    if not nm.m("tome_dot_not_cos"):
        sim = sim / np.maximum(np.linalg.norm(A, axis=1), 1e-9)[:, None]
        sim = sim / np.maximum(np.linalg.norm(B, axis=1), 1e-9)[None, :]
    best_b = np.argmax(sim, axis=1)
    best = sim[np.arange(n_a), best_b]
    order = sorted(range(n_a), key=lambda a: (best[a] if nm.m("tome_merge_lowest") else -best[a], a))
    chosen = set(order[:r])
    merged = [B[b].copy() for b in range(n_b)]
    count = [1] * n_b
    for a in range(n_a):
        if a in chosen:
            merged[best_b[a]] = merged[best_b[a]] + A[a]
            count[best_b[a]] += 1
    if not nm.m("tome_no_average"):
        merged = [merged[b] / count[b] for b in range(n_b)]
    umap = np.zeros(seq, np.int64)
    umap[1::2] = np.arange(n_b)
    kept = []
    for a in range(n_a):
        if a in chosen:
            umap[2 * a] = best_b[a]
        else:
            umap[2 * a] = n_b + len(kept)
            kept.append(A[a])
    out = np.array(merged + kept).reshape(seq - r, x.shape[1])
    sb = np.sort(best)[::-1]
    second = np.sort(sim, axis=1)[:, -2] if n_b > 1 else best - 1.0
    info = {"rank_margin": float(sb[r - 1] - sb[r]) if 0 < r < n_a else float("inf"),
            "edge_margin": float(np.min((best - second)[sorted(chosen)])) if chosen else float("inf"),
            "umap": umap.copy()}
    return out, umap, info


class Encoder:
    """Whisper audio encoder: two GELU convs (k=3, pad 1; strides 1, 2), sinusoid
    slot filled by the file's positional embedding, pre-LN transformer blocks,
    final LayerNorm."""

    def __init__(self, model, nm: Numerics | None = None):
        self.t, self.cfg = model.t, model.cfg
        self.nm = nm or Numerics()

    def _g(self, name):
        a = self.t[name]
        return w16(a) if a.dtype == np.uint16 else np.asarray(a, np.float64)

    def conv(self, x, wname, bname, stride):
        w = self._g(wname)  # [out, in, 3]
        if self.nm.m("conv_taps_reversed"):
            w = w[:, :, ::-1]
        b = self._g(bname)
        t_in = x.shape[0]
        xp = np.concatenate([np.zeros((1, x.shape[1])), x, np.zeros((1, x.shape[1]))])
        t_out = (t_in + 2 - 3) // stride + 1
        start = 1 if (stride == 2 and self.nm.m("conv2_stride1_even")) else 0
        out = np.tile(b, (t_out, 1))
        for kk in range(3):
            rows = xp[start + kk: start + kk + stride * t_out: stride]
            if rows.shape[0] < t_out:
                rows = np.concatenate([rows, np.zeros((t_out - rows.shape[0], x.shape[1]))])
            out += rows @ w[:, :, kk].T
        return out

    def linear(self, x, p, bias=True):
        y = x @ self._g(p + ".weight").T
        if bias:
            y = y + self._g(p + ".bias")
        return y

    def block(self, x, i):
        nm, p = self.nm, f"encoder.blocks.{i}"
        h = nm.ln(x, self._g(p + ".attn_ln.weight"), self._g(p + ".attn_ln.bias"))
        q = self.linear(h, p + ".attn.query", bias=not nm.m("no_q_bias"))
        k = self.linear(h, p + ".attn.key", bias=False)
        if nm.m("k_bias_from_q"):
            k = k + self._g(p + ".attn.query.bias")
        v = self.linear(h, p + ".attn.value", bias=not nm.m("no_v_bias"))
        a = mha(q, k, v, self.cfg.n_audio_head, nm)
        x = x + self.linear(a, p + ".attn.out", bias=not nm.m("no_o_bias"))
        h = nm.ln(x, self._g(p + ".mlp_ln.weight"), self._g(p + ".mlp_ln.bias"))
        f = nm.gelu(self.linear(h, p + ".mlp.0", bias=not nm.m("no_fc1_bias")))
        return x + self.linear(f, p + ".mlp.2", bias=not nm.m("no_fc2_bias"))

    def forward(self, mel_time_major, n_layers=None, tome_r=0, tome_after=3, info=None, tome_every=0,
                tome_floor=128):
        """With tome_every > 0 the merge repeats after every tome_every blocks
        from tome_after on (the ToMe paper's progressive schedule) while the
        merged length stays >= tome_floor; the unmerge broadcasts each final
        row to every original row that was merged into it."""
        nm = self.nm
        x = np.asarray(mel_time_major, np.float64)
        x = nm.gelu(self.conv(x, "encoder.conv1.weight", "encoder.conv1.bias", 1))
        x = nm.gelu(self.conv(x, "encoder.conv2.weight", "encoder.conv2.bias", 2))
        if not nm.m("no_pos_emb"):
            x = x + self._g("encoder.positional_embedding")[: x.shape[0]]
        L = self.cfg.n_audio_layer if n_layers is None else n_layers
        umap = None
        n_merges = 0
        floor = 0 if nm.m("tome_ignore_floor") else tome_floor
        phase = 1 if nm.m("tome_every_off_by_one") else 0
        for i in range(L):
            x = self.block(x, i)
            due = (umap is None and i == tome_after) if tome_every == 0 else \
                (i >= tome_after and (i - tome_after) % tome_every == phase)
            if tome_r > 0 and due and x.shape[0] > tome_r + 2 and x.shape[0] - tome_r >= floor:
                x, step, tinfo = tome_merge(x, tome_r, nm)
                umap = step if umap is None else step[umap]  # original row -> current row
                n_merges += 1
                if info is not None:
                    info["rank_margin"] = min(info.get("rank_margin", np.inf), tinfo["rank_margin"])
                    info["edge_margin"] = min(info.get("edge_margin", np.inf), tinfo["edge_margin"])
                    info["merges"] = n_merges
        if umap is not None:
            x = x[umap]
        if nm.m("no_ln_post"):
            return x
        return nm.ln(x, self._g("encoder.ln_post.weight"), self._g("encoder.ln_post.bias"))


class Decoder:
    """Whisper text decoder: token + learned positional embedding, pre-LN blocks
    of causal self-attention, cross-attention over the encoder states and a GELU
    MLP, final LayerNorm, logits against the (tied) token embedding."""

    def __init__(self, model, nm: Numerics | None = None):
        self.t, self.cfg = model.t, model.cfg
        self.nm = nm or Numerics()

    def _g(self, name):
        a = self.t[name]
        return w16(a) if a.dtype == np.uint16 else np.asarray(a, np.float64)

    def linear(self, x, p, bias=True):
        y = x @ self._g(p + ".weight").T
        if bias:
            y = y + self._g(p + ".bias")
        return y

    def state(self, enc):
        return DecoderState(self, np.asarray(enc, np.float64))


class DecoderState:
    def __init__(self, dec: Decoder, enc):
        self.dec, self.nm = dec, dec.nm
        cfg = dec.cfg
        nm = self.nm
        self.ck, self.cv = [], []
        for i in range(cfg.n_text_layer):
            p = f"decoder.blocks.{i}.cross_attn"
            k = dec.linear(enc, p + ".key", bias=False)
            v = dec.linear(enc, p + ".value", bias=not nm.m("no_cross_v_bias"))
            if nm.cross_f16:
                # the cache holds k * d_head^-1/4 (and q is scaled the same way at
                # use), each rounded to f16
                s4 = (cfg.n_text_state // cfg.n_text_head) ** -0.25
                k, v = f16(k * s4) / s4, f16(v)
            self.ck.append(k)
            self.cv.append(v)
        self.kc = [np.zeros((0, cfg.n_text_state)) for _ in range(cfg.n_text_layer)]
        self.vc = [np.zeros((0, cfg.n_text_state)) for _ in range(cfg.n_text_layer)]
        self.len = 0

    def step(self, tokens):
        """Feed tokens (one or a prompt); return the last row's logits."""
        dec, nm, cfg = self.dec, self.nm, self.dec.cfg
        tokens = np.asarray(tokens, np.int64).ravel()
        tq = tokens.size
        pos = np.arange(self.len, self.len + tq)
        if nm.m("pos_emb_shift"):
            pos = pos + 1
        x = dec._g("decoder.token_embedding.weight")[tokens] + dec._g("decoder.positional_embedding")[pos]
        H = cfg.n_text_head
        for i in range(cfg.n_text_layer):
            p = f"decoder.blocks.{i}"
            h = nm.ln(x, dec._g(p + ".attn_ln.weight"), dec._g(p + ".attn_ln.bias"))
            q = dec.linear(h, p + ".attn.query", bias=not nm.m("no_q_bias"))
            k = dec.linear(h, p + ".attn.key", bias=False)
            if nm.m("k_bias_from_q"):
                k = k + dec._g(p + ".attn.query.bias")
            v = dec.linear(h, p + ".attn.value", bias=not nm.m("no_v_bias"))
            if nm.kv_f16:
                k, v = f16(k), f16(v)
            self.kc[i] = np.concatenate([self.kc[i], k])
            self.vc[i] = np.concatenate([self.vc[i], v])
            a = mha(q, self.kc[i], self.vc[i], H, nm, causal_offset=self.len)
            x = x + dec.linear(a, p + ".attn.out", bias=not nm.m("no_o_bias"))
            h = nm.ln(x, dec._g(p + ".cross_attn_ln.weight"), dec._g(p + ".cross_attn_ln.bias"))
            q = dec.linear(h, p + ".cross_attn.query")
            if nm.m("cross_k_unscaled"):
                a = mha(q * np.sqrt(cfg.n_text_state // H), self.ck[i], self.cv[i], H, nm)
            else:
                a = mha(q, self.ck[i], self.cv[i], H, nm)
            x = x + dec.linear(a, p + ".cross_attn.out")
            h = nm.ln(x, dec._g(p + ".mlp_ln.weight"), dec._g(p + ".mlp_ln.bias"))
            f = nm.gelu(dec.linear(h, p + ".mlp.0", bias=not nm.m("no_fc1_bias")))
            x = x + dec.linear(f, p + ".mlp.2", bias=not nm.m("no_fc2_bias"))
        self.len += tq
        h = x[-1]
        if not nm.m("no_final_ln"):
            h = nm.ln(h, dec._g("decoder.ln.weight"), dec._g("decoder.ln.bias"))
        return dec._g("decoder.token_embedding.weight") @ h

    def greedy(self, prompt, n_max, suppress):
        """Greedy no-timestamps loop: sample from the prompt's logits, feed each
        sampled token back, stop after end-of-text or n_max samples.
        `suppress(logits, first)` returns the masked logits."""
        logits = self.step(prompt)
        out = []
        eot = suppress.eot
        for i in range(n_max):
            tok = int(np.argmax(suppress(logits, i == 0)))
            out.append(tok)
            if tok == eot or i + 1 == n_max:
                break
            logits = self.step([tok])
        return np.array(out, np.int32)


class NoTimestampsFilter:
    """The no-timestamps logit filter of Whisper's decoding: suppress the special
    tokens (sot, sot_prev, solm, no_speech, no_timestamps, translate, transcribe,
    every language token), every timestamp token, and on the first sampled step
    end-of-text and the blank token."""

    def __init__(self, tokens, n_vocab, n_languages=100):
        self.eot = tokens.eot
        ids = [tokens.sot, tokens.sot_prev, tokens.solm, tokens.no_speech, tokens.no_timestamps,
               tokens.translate, tokens.transcribe]
        ids += [tokens.sot + 1 + i for i in range(n_languages)]
        self.mask = np.zeros(n_vocab, bool)
        self.mask[[i for i in ids if 0 <= i < n_vocab]] = True
        self.mask[tokens.timestamp_begin:] = True
        self.first = [tokens.eot, tokens.space]

    def __call__(self, logits, first):
        lg = np.where(self.mask, -np.inf, logits)
        if first:
            lg = lg.copy()
            lg[self.first] = -np.inf
        return lg
