"""CPU restatement of the multi-block slot plan that plan_kernel / place_kernel compute on the GPU
(csrc/route.hip; reference engine/ops.cu:384-423), checked against the oracle's counting sort (orc_dispatch).

The GPU planner gives thread e the expert e and scans over the 256 experts in two levels: an inclusive scan inside
each 64-lane wave, then the totals of the lower waves added from LDS. Slot bases per (block, expert) follow from
the per-block token masks. Restating exactly those two levels here pins the arithmetic the kernel implements,
and the negative case shows that a wave reading a wrong wave total (the failure mode of an LDS race on the
wave-total array) changes slot_token, so the GPU test on the same routing detects it.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from llmoe import synth


def _masks(topk, block, E):
    T, K = topk.shape
    nb = (T + block - 1) // block
    mask = np.zeros((nb, E), np.uint64)
    for t in range(T):
        for k in range(K):
            mask[t // block, topk[t, k]] |= np.uint64(1) << np.uint64(t % block)
    return mask


def _popc(a):
    a = np.asarray(a, np.uint64)
    return np.array([bin(int(v)).count("1") for v in a.ravel()], np.int64).reshape(a.shape)


def _two_level_excl_scan(c, wave_total_override=None):
    """Exclusive scan over experts as the planner does it: per-wave inclusive scans, then lower-wave totals.
    wave_total_override(w, totals) may replace the totals a wave reads (to model a corrupted LDS entry)."""
    E = c.size
    incl = np.zeros(E, np.int64)
    totals = []
    for w0 in range(0, E, 64):
        seg = np.cumsum(c[w0:w0 + 64])
        incl[w0:w0 + 64] = seg
        totals.append(int(seg[-1]))
    for w in range(len(totals)):
        seen = totals if wave_total_override is None else wave_total_override(w, totals)
        incl[w * 64:(w + 1) * 64] += sum(seen[:w])
    return incl - c


def plan_place(topk, topw, E, block, has_shared, wave_total_override=None):
    T, K = topk.shape
    mask = _masks(topk, block, E)
    pc = _popc(mask)                                   # [nb, E]
    count = pc.sum(axis=0)
    start = _two_level_excl_scan(count, wave_total_override)
    bpre = start[None, :] + np.cumsum(pc, axis=0) - pc  # slot base of each (block, expert)
    S = T * K + (T if has_shared else 0)
    slot_token = np.zeros(S, np.int32)
    slot_weight = np.zeros(S, np.float32)
    tok_slots = np.zeros((T, K + 1), np.int32)
    for t in range(T):
        b, tl = divmod(t, block)
        for k in range(K):
            ex = topk[t, k]
            below = int(mask[b, ex]) & ((1 << tl) - 1)
            sl = int(bpre[b, ex]) + bin(below).count("1")
            slot_token[sl] = t
            slot_weight[sl] = topw[t, k]
            tok_slots[t, k] = sl
        tok_slots[t, K] = T * K + t if has_shared else -1
        if has_shared:
            slot_token[T * K + t] = t
            slot_weight[T * K + t] = 1.0
    return dict(count=count.astype(np.int32), start=start.astype(np.int32), slot_token=slot_token,
                slot_weight=slot_weight, tok_slots=tok_slots)


def _routing(T, kind, E=256):
    lg = synth.logits_zipf(T + 1, T, E) if kind == "zipf" else synth.logits_skewed(T + 1, T, E)
    bias = np.random.default_rng(7).uniform(-0.1, 0.1, E).astype(np.float32)
    return O.route(lg, bias, K=8, C=256)


@pytest.mark.parametrize("T,kind,shared", [(512, "skewed", True), (300, "skewed", False), (256, "zipf", True),
                                           (33, "zipf", True)])
def test_plan_restatement_matches_oracle_dispatch(T, kind, shared):
    topk, topw = _routing(T, kind)
    want = O.dispatch(topk, topw, 256, shared)
    got = plan_place(topk, topw, 256, 32, shared)
    for key in ("count", "start", "slot_token", "tok_slots"):
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    np.testing.assert_array_equal(got["slot_weight"].view(np.uint32), want["slot_weight"].view(np.uint32))


def test_corrupted_wave_total_changes_slot_token():
    """A wave that reads the chunk count in place of wave 0's slot total misplaces slots (T=512, skewed)."""
    topk, topw = _routing(512, "skewed")
    want = O.dispatch(topk, topw, 256, True)
    bad = plan_place(topk, topw, 256, 32, True,
                     wave_total_override=lambda w, tot: [tot[0] // 7] + tot[1:] if w in (1, 2) else tot)
    assert not np.array_equal(bad["slot_token"], want["slot_token"])
