"""The 16-layer decoder at its full configuration (d_model 1024, 8 heads of
128, MLP 4096 ReLU², vocabulary 50304, bf16; window 4 blocks of 128, budget
4, one global block).  Its model glue mirrors GPT.forward
(scoped_medium.py:578-639), whose module cannot be imported (it initialises
CUDA, NCCL and an 8-rank world at import), so its logits stay parity
unpinned against the reference; these are the size-independent properties
of the token loop at the full size:

* after a 131072-token prefill, the decode steps that replay the captured
  HIP graph give the logits of the eager steps (same operations; |Δ| <= 1e-6),
  across two q-block starts;
* the token loop equals the prefill of the whole sequence at every position
  where both attend over the same key blocks: a 512-token prompt (4 blocks),
  then 130 steps across the block starts at 512 and 640 with documents
  opening before and inside the loop.  There window 4 + the global block
  cover every candidate block, so the per-block reselection has nothing to
  choose and both paths list the same blocks.  Logits |step - prefill| <=
  5e-2 (the logits are 30·σ(x/7.5), in [0, 30]); the argmax agrees wherever
  the prefill's top-two gap exceeds twice that bar.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model(max_len: int, use_graph: bool):
    from scope_amd.decode import DecoderConfig, ScopeDecoder

    return ScopeDecoder(DecoderConfig(), max_len=max_len, device=DEV, seed=0, use_graph=use_graph)


def test_c4_graph_steps_equal_eager_after_long_prefill():
    T0, n = 131072, 140
    g = torch.Generator().manual_seed(0)
    toks = torch.randint(0, 50257, (T0 + n,), generator=g)
    toks[[77777, T0 + 60]] = 50256  # a document opens in the prompt and one inside the loop
    cap = T0 + 2 * 128
    print(f"16-layer decoder: prefill {T0} tokens twice, {n} steps graph vs eager", flush=True)
    eager = _model(cap, use_graph=False)
    graph = _model(cap, use_graph=True)
    la = eager.prefill(toks[:T0])
    lb = graph.prefill(toks[:T0])
    torch.cuda.synchronize()
    assert torch.equal(la, lb)
    worst = 0.0
    for s_ in range(n):
        a = eager.step(toks[T0 + s_])
        b = graph.step(toks[T0 + s_])
        torch.cuda.synchronize()
        d = (a - b).abs().max().item()
        worst = max(worst, d)
        assert d <= 1e-6, f"position {T0 + s_}: |graph - eager| = {d:.3e}"
        assert int(a.argmax()) == int(b.argmax())
    assert graph._graph is not None, "no step ran as a graph"
    assert torch.equal(eager.docs[:T0 + n], graph.docs[:T0 + n])
    print(f"  max |graph - eager| {worst:.3e}", flush=True)


def test_c4_token_loop_matches_prefill_full_config():
    T0, n, Tp = 512, 130, 768
    g = torch.Generator().manual_seed(3)
    toks = torch.randint(0, 50257, (Tp,), generator=g)
    toks[[50, 300, 450, 600]] = 50256
    print("16-layer decoder: token loop vs prefill", flush=True)
    m = _model(1024, use_graph=True)
    m.prefill(toks[:T0])
    got = torch.stack([m.step(toks[T0 + s]) for s in range(n)])
    full = _model(1024, use_graph=False)
    ref = full.prefill(toks[:Tp], all_logits=True)[T0:T0 + n]
    err = (got - ref).abs().max().item()
    print(f"  max |step - prefill| logit diff {err:.3e}", flush=True)
    assert err <= 5e-2, f"max logit difference {err:.3e}"
    top2 = ref.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * 5e-2
    agree = got.argmax(-1) == ref.argmax(-1)
    assert bool(agree[clear].all()), f"argmax differs at clear positions {torch.nonzero(clear & ~agree).flatten()}"
    print(f"  argmax agrees at {int(agree.sum())}/{n} positions ({int(clear.sum())} with a clear top-two gap)",
          flush=True)
