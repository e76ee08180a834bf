"""Pins the oracle's layer wiring (which activation feeds which stage, which side of each weight is
multiplied) that the primitive pins and invariants leave open.

1. An independent fp64 restatement of one layer, written from the stage list of the reference's kernel
   (src/mk_expert.py:342-419: AdaRMS -> q/k/v, per-head q/k RMSNorm + rotate-half RoPE, self-attention over
   [memory rows kv_start..PM || own rows], out-projection with the SA gate, AdaRMS of h2 -> CA query, CA over
   the S valid source rows, CA out-projection with its gate, AdaRMS of h3 -> gated MLP, down-projection with
   the MLP gate) with torch.nn.functional.linear / rms_norm / scaled_dot_product_attention and boolean key
   masks (not the oracle's row slicing), against ``expert_ref.layer_forward`` on random non-symmetric weights
   and random modulation rows (every gate non-zero).
2. Mutants of ``layer_forward`` (a transposed square projection; h instead of h2 or h3 into an AdaRMS), planted
   in a copy of the oracle on the CPU: the independent restatement must tell each of them apart.
3. A structured probe: with a cyclic-shift out-projection S (S[i, j] = 1 iff j = i + 1 mod H) and only that
   stage's gate open, the layer adds y[:, i + 1] to column i — a transposed product would add y[:, i - 1].
"""
import inspect

import pytest
import torch
import torch.nn.functional as F

from oracle import expert_ref as ER

D = ER.ExpertDims(L=1, H=128, NH=2, HD=64, I=256, A=32, ctx_dim=64, tdim=32, eps=1e-6, qk_eps=1e-6, act="silu")
M, PM, KVS, SP, S_LEN = 7, 10, 3, 12, 9


def _case(seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=1.0: torch.randn(*s, generator=g, dtype=torch.float64) * sc  # noqa: E731
    H, I, HD, NH = D.H, D.I, D.HD, D.NH
    lw = {"q": r(H, H, sc=0.1), "k": r(H, H, sc=0.1), "v": r(H, H, sc=0.1), "o": r(H, H, sc=0.1),
          "ca_q": r(H, H, sc=0.1), "ca_o": r(H, H, sc=0.1), "gate": r(I, H, sc=0.1), "up": r(I, H, sc=0.1),
          "down": r(H, I, sc=0.1), "q_norm": r(HD, sc=0.2), "k_norm": r(HD, sc=0.2), "ca_q_norm": r(HD, sc=0.2)}
    W = {"layers": [lw]}
    ang = r(M, HD // 2)
    cos, sin = torch.cos(torch.cat([ang, ang], -1)), torch.sin(torch.cat([ang, ang], -1))
    cang = r(M, HD // 2)
    ccos, csin = torch.cos(torch.cat([cang, cang], -1)), torch.sin(torch.cat([cang, cang], -1))
    cache = {"sa_cos": cos, "sa_sin": sin, "ca_cos": ccos, "ca_sin": csin,
             "memk": r(1, 1, PM, NH, HD), "memv": r(1, 1, PM, NH, HD), "kv_start": torch.tensor([KVS]),
             "kca": r(1, 1, SP, NH, HD), "vca": r(1, 1, SP, NH, HD), "ca_len": torch.tensor([S_LEN])}
    mrow = r(D.modw, sc=0.5)
    h = r(M, H)
    return h, W, mrow, cache


def _rope(x, cos, sin):
    # rotate-half RoPE of [rows, NH, HD] with tables [rows, HD]
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return x * cos[:, None, :] + torch.cat([-x2, x1], -1) * sin[:, None, :]


def independent_layer(h, W, mrow, cache):
    """One layer, fp64, restated from the kernel's stage list with torch.nn.functional primitives."""
    H, NH, HD = D.H, D.NH, D.HD
    lw = W["layers"][0]
    blocks = mrow[: 9 * H].view(9, H)  # [sa scale, sa shift, sa gate, ca scale, ca shift, ca gate, mlp ...]
    ada = lambda x, sc, sh: F.rms_norm(x, (H,), eps=D.eps) * (1 + sc) + sh  # noqa: E731
    qkn = lambda x, w: F.rms_norm(x, (HD,), weight=1 + w, eps=D.qk_eps)  # noqa: E731

    def attention(q, k, v, valid):
        # q [Mq, NH, HD], k / v [N, NH, HD], valid [N] bool: every query attends to the valid keys
        out = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                             attn_mask=valid[None, None, :].expand(NH, q.shape[0], -1))
        return out.transpose(0, 1).reshape(q.shape[0], H)

    a = ada(h, blocks[0], blocks[1])
    q = F.linear(a, lw["q"]).view(M, NH, HD)
    k = F.linear(a, lw["k"]).view(M, NH, HD)
    v = F.linear(a, lw["v"]).view(M, NH, HD)
    q = _rope(qkn(q, lw["q_norm"]), cache["sa_cos"], cache["sa_sin"])
    k = _rope(qkn(k, lw["k_norm"]), cache["sa_cos"], cache["sa_sin"])
    keys = torch.cat([cache["memk"][0, 0], k], 0)
    vals = torch.cat([cache["memv"][0, 0], v], 0)
    valid = torch.cat([torch.arange(PM) >= int(cache["kv_start"][0]), torch.ones(M, dtype=torch.bool)])
    h2 = h + F.linear(attention(q, keys, vals, valid), lw["o"]) * blocks[2]
    a = ada(h2, blocks[3], blocks[4])
    qc = _rope(qkn(F.linear(a, lw["ca_q"]).view(M, NH, HD), lw["ca_q_norm"]), cache["ca_cos"], cache["ca_sin"])
    valid = torch.arange(SP) < int(cache["ca_len"][0])
    h3 = h2 + F.linear(attention(qc, cache["kca"][0, 0], cache["vca"][0, 0], valid), lw["ca_o"]) * blocks[5]
    a = ada(h3, blocks[6], blocks[7])
    g = F.silu(F.linear(a, lw["gate"])) * F.linear(a, lw["up"])
    return h3 + F.linear(g, lw["down"]) * blocks[8]


def _oracle(fn, h, W, mrow, cache):
    return fn(h, 0, W, mrow, cache, 0, D, "fp64")


def test_layer_matches_an_independent_restatement():
    for seed in range(3):
        h, W, mrow, cache = _case(seed)
        ref = independent_layer(h, W, mrow, cache)
        got = _oracle(ER.layer_forward, h, W, mrow, cache)
        assert (got - ref).abs().max().item() < 1e-10, seed
        assert (got - h).abs().max().item() > 1e-2  # the layer does change h


def _mutant(old: str, new: str):
    src = inspect.getsource(ER.layer_forward)
    assert src.count(old) == 1, old
    ns = dict(vars(ER))
    exec(compile(src.replace(old, new), "<mutant>", "exec"), ns)
    return ns["layer_forward"]


@pytest.mark.parametrize("old,new", [
    ('Rr(Q(y) @ lw["o"].T)', 'Rr(Q(y) @ lw["o"])'),          # transposed self-attention out-projection
    ('Rr(Q(y) @ lw["ca_o"].T)', 'Rr(Q(y) @ lw["ca_o"])'),    # transposed cross-attention out-projection
    ('R(a @ lw["ca_q"].T)', 'R(a @ lw["ca_q"])'),      # transposed cross-attention query projection
    ('R(a @ lw["q"].T)', 'R(a @ lw["q"])'),            # transposed q projection
    ("a = ada(h2, ca_sc", "a = ada(h, ca_sc"),          # CA query from h instead of h2
    ("a = ada(h3, m_sc", "a = ada(h2, m_sc"),           # MLP from h2 instead of h3
    ("h3 = Rr(h2 +", "h3 = Rr(h +"),                   # CA residual onto h instead of h2
])
def test_planted_wiring_mistakes_are_detected(old, new):
    mutant = _mutant(old, new)
    h, W, mrow, cache = _case(0)
    ref = independent_layer(h, W, mrow, cache)
    assert (_oracle(mutant, h, W, mrow, cache) - ref).abs().max().item() > 1e-4


def _only_gate(mrow, which):
    m = mrow.clone()
    H = D.H
    for blk in (2, 5, 8):  # sa, ca, mlp gates
        m[blk * H:(blk + 1) * H] = 1.0 if blk == which else 0.0
    return m


@pytest.mark.parametrize("wname,gate", [("o", 2), ("ca_o", 5)])
def test_shift_projection_lands_on_the_next_column(wname, gate):
    h, W, mrow, cache = _case(1)
    m = _only_gate(mrow, gate)
    H = D.H
    eye = torch.eye(H, dtype=torch.float64)
    shift = torch.roll(eye, 1, dims=1)  # shift[i, j] = 1 iff j == i + 1 (mod H)
    W["layers"][0][wname] = eye
    y = _oracle(ER.layer_forward, h, W, m, cache) - h  # the stage's output itself (identity projection)
    W["layers"][0][wname] = shift
    out = _oracle(ER.layer_forward, h, W, m, cache) - h
    assert torch.allclose(out, torch.roll(y, -1, dims=1), atol=1e-12)  # column i receives y[:, i + 1]
    assert not torch.allclose(out, torch.roll(y, 1, dims=1), atol=1e-6)
