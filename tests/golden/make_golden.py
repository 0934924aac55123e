"""Writes the golden fixtures of tests/golden/*.npz (run: python tests/golden/make_golden.py).

The reference repository ships no tests, fixtures or golden vectors, so these vectors come
from the libraries the reference calls and from closed forms, generated in this container:
  topk_*.npz     torch.softmax + torch.topk on the CPU (the calls of ferry/model.py:142-146 and
                 the HF DeepSeek-V2 gate), tie-heavy rows included;
  layout.npz     numpy stable argsort / bincount / cumsum (closed form of ferry/layout.py:12-94
                 at world = 1), cross-checked against the literal loop restatement;
  history.npz    the ring restatement of ferry/metadata.py:15-38, cross-checked against the
                 closed form (counts over the last min(W, seen) tokens);
  planner.npz    plan_layer at world = 1 (ferry/policy.py:130-194), cross-checked between the C
                 restatement and the sort-based formulation.
"""
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.history import GateHistoryRef, closed_form_scores, frequency_rows  # noqa: E402
from oracle.layout import layout_closed_form, layout_loops  # noqa: E402
from oracle.policy import PlannerRef, plan_layer_sorted  # noqa: E402


def topk_fixtures():
    g = torch.Generator().manual_seed(2024)
    # Qwen3 router: bf16 logits, coarse values -> ties at every position
    z = torch.randn((512, 128), generator=g)
    z[:256] = torch.round(z[:256] * 4) / 4
    logits = z.to(torch.bfloat16)
    probs = torch.softmax(logits, dim=-1, dtype=torch.float32)
    w, idx = torch.topk(probs, 8, dim=-1)
    w = (w / w.sum(-1, keepdim=True)).to(torch.bfloat16)
    np.savez_compressed(HERE / 'topk_qwen3_bf16.npz', logits=logits.view(torch.int16).numpy(),
                        idx=idx.numpy(), w=w.view(torch.int16).numpy(), k=8)
    # DeepSeek-V2 gate: fp32 logits, topk(sorted=False)
    z = torch.randn((512, 64), generator=g)
    z[::2] = torch.round(z[::2] * 3) / 3
    probs = torch.softmax(z, dim=-1)
    w, idx = torch.topk(probs, 6, dim=-1, sorted=False)
    np.savez_compressed(HERE / 'topk_deepseek_fp32_unsorted.npz', logits=z.numpy(), idx=idx.numpy(),
                        w=w.to(torch.bfloat16).view(torch.int16).numpy(), k=6)


def layout_fixture():
    rng = np.random.default_rng(7)
    T, E, k = 300, 128, 8
    sel = np.stack([rng.choice(E, k, replace=False, p=None) for _ in range(T)]).astype(np.int64)
    ref = layout_closed_form(sel, E)
    loops = layout_loops(sel, E)
    for key in ('send_ids', 'starts', 'rows', 'cols'):
        assert np.array_equal(ref[key], loops[key]), key
    np.savez_compressed(HERE / 'layout.npz', selected=sel, experts=E, send_ids=ref['send_ids'],
                        starts=ref['starts'], rows=ref['rows'], cols=ref['cols'],
                        pair_pos=ref['pair_pos'])


def history_fixture():
    rng = np.random.default_rng(11)
    L, E, k, W = 2, 32, 4, 16
    h = GateHistoryRef(L, E, W)
    seen = [[] for _ in range(L)]
    sizes = [3, 5, 20, 1, 7, 16, 2, 9, 15, 1, 30, 4]
    calls, scores = [], []
    for i, T in enumerate(sizes):
        layer = i % L
        sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
        h.update(layer, frequency_rows(sel, E, W))
        seen[layer].extend(list(sel))
        s = h.scores(layer)
        assert np.array_equal(s, closed_form_scores(seen[layer], E, W))
        calls.append(sel)
        scores.append(s)
    np.savez_compressed(HERE / 'history.npz', sizes=np.array(sizes), layers=L, experts=E, topk=k,
                        window=W, selected=np.concatenate(calls), scores=np.stack(scores))


def planner_fixture():
    rng = np.random.default_rng(5)
    L, E, cap, k = 3, 16, 9, 3
    ref = PlannerRef(L, E, cap)
    st = dict(slots=np.full(cap, -1, np.int64), owner=np.full(L * E, -1, np.int64),
              last=np.zeros(L * E, np.int64), scores=np.zeros((L, E), np.float32))
    sizes, sels, gss, fetches = [], [], [], []
    for ev in range(60):
        layer = ev % L
        T = int(rng.integers(1, 4))
        sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
        gs = (rng.integers(0, 4, E) / 4).astype(np.float32)   # coarse scores: many ties
        f1, _ = ref.plan(ev, layer, sel, gs)
        f2 = plan_layer_sorted(st, ev, layer, sel, gs)
        assert np.array_equal(f1, f2), ev
        sizes.append(T)
        sels.append(sel)
        gss.append(gs)
        fetches.append(f1)
    np.savez_compressed(HERE / 'planner.npz', layers=L, experts=E, cap=cap, topk=k,
                        sizes=np.array(sizes), selected=np.concatenate(sels), gate_scores=np.stack(gss),
                        nfetch=np.array([len(f) for f in fetches]),
                        fetches=np.concatenate(fetches).reshape(-1, 3), final_slots=ref.slots,
                        final_last=ref.last)


if __name__ == '__main__':
    topk_fixtures()
    layout_fixture()
    history_fixture()
    planner_fixture()
    print('fixtures written to', HERE)
