"""The oracle's layer restatement and error bound, pinned on the CPU: the float64 exact result against a per-element
sum written independently, the restatements within their own rounding distance of exact, and planted mistakes
(a dropped LoRA term, a transposed factor, a wrong adapter) caught by the bound."""

from __future__ import annotations

import numpy as np
import torch

from oracle.layer import (exact_and_bound, layer_float32, layer_model, reference_f32, uncut_bound,
                          within_tolerance)


def small_case(seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    t, k, cols, r = 12, 64, [16, 8], 4
    x = torch.randn(t, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(sum(cols), k, generator=g) * 0.05).to(torch.bfloat16)
    adapters = {a: [((torch.randn(r, k, generator=g) / 8).to(torch.bfloat16),
                     (torch.randn(n, r, generator=g) * 0.04).to(torch.bfloat16)) for n in cols] for a in (1, 2)}
    adapters[2][1] = None                              # adapter 2 does not adapt the second matrix
    token_adp = np.array([1, 1, 0, 2, 2, 2, 1, 0, 0, 2, 1, 1])
    return x, w, token_adp, adapters, cols, r


def per_element_exact(x, w, token_adp, adapters, cols):
    t, k = x.shape
    edges = np.concatenate([[0], np.cumsum(cols)])
    out = np.zeros((t, sum(cols)))
    xd, wd = x.double().numpy(), w.double().numpy()
    for i in range(t):
        for o in range(sum(cols)):
            v = sum(xd[i, q] * wd[o, q] for q in range(k))
            j = int(np.searchsorted(edges, o, side="right") - 1)
            upd = adapters.get(int(token_adp[i]), [None] * len(cols))[j] if int(token_adp[i]) in adapters else None
            if upd is not None:
                a_mat, sb = (m.double().numpy() for m in upd)
                for rr in range(a_mat.shape[0]):
                    v += sum(xd[i, q] * a_mat[rr, q] for q in range(k)) * sb[o - edges[j], rr]
            out[i, o] = v
    return out


def test_exact_equals_an_independent_per_element_sum() -> None:
    x, w, tok, adapters, cols, r = small_case()
    exact, bound = exact_and_bound(x, w, tok, adapters, cols, r * 2)
    want = per_element_exact(x, w, tok, adapters, cols)
    assert np.allclose(exact.numpy(), want, rtol=0, atol=1e-12)
    assert (bound > 0).all()


def test_restatements_sit_within_their_rounding_of_exact() -> None:
    x, w, tok, adapters, cols, r = small_case(1)
    exact, bound = exact_and_bound(x, w, tok, adapters, cols, r * 2)
    f32 = reference_f32(x, w, tok, adapters, cols).double()
    assert ((f32 - exact).abs() <= bound).all()
    once = f32.float().to(torch.bfloat16).double()               # one rounding of a float32 result: inside the bound
    assert ((once - exact).abs() <= bound).all()
    model = layer_model(x, w, tok, adapters, cols).double()     # rounds the base, then the sum: the uncut bound
    assert ((model - exact).abs() <= uncut_bound(x, w, exact, bound)).all()
    assert within_tolerance(layer_float32(x, w, tok, adapters, cols), f32.float()).all()


def test_planted_mistakes_are_caught_by_the_bound() -> None:
    x, w, tok, adapters, cols, r = small_case(2)
    exact, bound = exact_and_bound(x, w, tok, adapters, cols, r * 2)

    def fails(bad_adapters=None, bad_tok=None, bad_w=None):
        got = reference_f32(x, bad_w if bad_w is not None else w, bad_tok if bad_tok is not None else tok,
                            bad_adapters if bad_adapters is not None else adapters, cols)
        return bool(((got.to(torch.bfloat16).double() - exact).abs() > bound).any())

    dropped = {a: [None] * len(cols) for a in adapters}
    assert fails(bad_adapters=dropped)
    swapped = {a: [None if u is None else (u[0].flip(0), u[1]) for u in ups] for a, ups in adapters.items()}
    assert fails(bad_adapters=swapped)
    assert fails(bad_tok=np.where(tok == 1, 2, tok))
    assert fails(bad_w=w.flip(1))


def test_planted_mistakes_are_caught_by_the_uncut_bound() -> None:
    """The uncut bound (a base rounded to bfloat16 before the LoRA update, as lora_add and the "model" precision
    round) admits the correct two-rounding restatement but not the same restatement with a plausible mistake: the
    LoRA term dropped or applied twice, A's rank rows reversed, another adapter's update, transposed weights."""
    x, w, tok, adapters, cols, r = small_case(3)
    exact, bound = exact_and_bound(x, w, tok, adapters, cols, r * 2)
    allowed = uncut_bound(x, w, exact, bound)
    assert ((layer_model(x, w, tok, adapters, cols).double() - exact).abs() <= allowed).all()

    def fails(bad_adapters=None, bad_tok=None, bad_w=None):
        got = layer_model(x, bad_w if bad_w is not None else w, bad_tok if bad_tok is not None else tok,
                          bad_adapters if bad_adapters is not None else adapters, cols)
        return bool(((got.double() - exact).abs() > allowed).any())

    assert fails(bad_adapters={a: [None] * len(cols) for a in adapters})
    assert fails(bad_adapters={a: [None if u is None else (u[0], (u[1].float() * 2).to(torch.bfloat16))
                                   for u in ups] for a, ups in adapters.items()})
    assert fails(bad_adapters={a: [None if u is None else (u[0].flip(0), u[1]) for u in ups]
                               for a, ups in adapters.items()})
    assert fails(bad_tok=np.where(tok == 1, 2, tok))
    assert fails(bad_w=w.flip(1))
