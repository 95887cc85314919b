"""Pins the oracle's per-expert packing (so_group) without restating its
linked list.

The reference groups selections by pushing idx = token*k + rank at the head
of its expert's list, skipping Weight <= 0 (forward/moe_batch.go:142-159),
so an expert's list holds its selections in descending idx, and lists are
laid out by ascending expert (forward/moe_schedule.go:25-101 walks experts
in order).  These tests check the oracle against facts that follow from
that definition and are computed differently here:
  - counts  == bincount of the expert ids of the kept selections
  - offsets == exclusive prefix sum of counts
  - every expert's slice is strictly descending and holds only its own idx
  - the union of the slices is exactly the set of kept idx (NaN weights are
    kept: NaN <= 0 is false)
  - the whole list equals a sort by (expert ascending, idx descending)
  - active == the experts with a non-empty list, ascending
and against a small case worked out by hand."""
import numpy as np
import pytest

from fixtures import ROUTER_MODES, moe_batch_fixture, moe_batch_x


def _check_group(O, ids, weights, batch, k, experts):
    ids = np.asarray(ids, np.int32)
    weights = np.asarray(weights, np.float32)
    counts, offsets, lst, active = O.group(ids, weights, batch, k, experts)
    kept = np.nonzero(~(weights <= 0))[0]  # NaN kept
    want_counts = np.bincount(ids[kept], minlength=experts).astype(np.int32)
    assert np.array_equal(counts, want_counts), "counts"
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts), "offsets"
    assert offsets[-1] == kept.size
    for e in range(experts):
        sl = lst[offsets[e]:offsets[e + 1]]
        assert np.all(np.diff(sl) < 0), f"expert {e} slice not strictly descending"
        assert np.all(ids[sl] == e), f"expert {e} slice holds another expert's idx"
    assert np.array_equal(np.sort(lst), kept), "union of slices != kept selections"
    order = np.lexsort((-kept, ids[kept]))  # primary: expert asc; secondary: idx desc
    assert np.array_equal(lst, kept[order]), "list != sort by (expert asc, idx desc)"
    assert np.array_equal(active, np.nonzero(want_counts)[0]), "active experts"
    return counts, offsets, lst, active


def test_group_hand_worked(O):
    # batch 4, k 2, experts 4.  Selections (idx: expert, weight):
    #   0: 2, .5   1: 0, .5   2: 2, .7   3: 1, 0 (skipped)
    #   4: 0, NaN (kept)  5: 2, .1   6: 3, -1 (skipped)  7: 0, .2
    ids = [2, 0, 2, 1, 0, 2, 3, 0]
    w = [.5, .5, .7, 0.0, np.nan, .1, -1.0, .2]
    counts, offsets, lst, active = O.group(np.array(ids, np.int32), np.array(w, np.float32), 4, 2, 4)
    assert counts.tolist() == [3, 0, 3, 0]
    assert offsets.tolist() == [0, 3, 3, 6, 6]
    assert lst.tolist() == [7, 4, 1, 5, 2, 0]  # pushed at head: last pushed first
    assert active.tolist() == [0, 2]
    # an ascending (push-at-tail) order would read [1, 4, 7, 0, 2, 5]
    assert lst.tolist() != [1, 4, 7, 0, 2, 5]
    _check_group(O, ids, w, 4, 2, 4)


@pytest.mark.parametrize("mode", ROUTER_MODES)
@pytest.mark.parametrize("experts,topk", [(1, 1), (4, 2), (7, 7), (8, 2)])
def test_group_router_modes(O, mode, experts, topk):
    """Selections of the reference fixture in every router mode (ties, NaN
    routers with fallback ids, the duplicate expert of mixed-nan, Inf
    routers with NaN weights, underflowed zero weights)."""
    lay = moe_batch_fixture(96, 64, experts, topk, 0, mode)
    rb = lay["router_bias"][0] if lay.get("router_bias") else np.zeros(experts, np.float32)
    for batch in (1, 5, 37):
        x = moe_batch_x(batch, 96, mode)
        logits = O.route(lay["router"], rb, x, batch, 96, experts)
        sel = [O.select(logits[t * experts:(t + 1) * experts], topk) for t in range(batch)]
        ids = np.concatenate([s[0] for s in sel])
        w = np.concatenate([s[1] for s in sel])
        _check_group(O, ids, w, batch, topk, experts)


@pytest.mark.parametrize("batch", [1, 8, 64, 512, 1024])
def test_group_gpt_oss_shape(O, batch):
    """128 experts, top-4: random expert ids (distinct within a token, as
    the top-k gives) with zero, negative and NaN weights mixed in."""
    rng = np.random.default_rng(batch)
    k, E = 4, 128
    ids = np.concatenate([rng.choice(E, k, replace=False) for _ in range(batch)]).astype(np.int32)
    w = rng.random(batch * k).astype(np.float32)
    drop = rng.random(batch * k)
    w[drop < 0.05] = 0.0
    w[(drop >= 0.05) & (drop < 0.08)] = np.nan
    w[(drop >= 0.08) & (drop < 0.10)] = -0.5
    _check_group(O, ids, w, batch, k, E)


def test_group_zipf_hot(O):
    """512 tokens, a quarter of them on one hot expert, the rest Zipf(1.1):
    one list of hundreds of entries beside many short ones."""
    from spt import synth

    batch, E, k = 512, 128, 4
    logits = synth.zipf_logits(synth.stream_key(4, 99), batch, E, 1.1, hot_fraction=0.25, hot_expert=17).reshape(-1)
    sel = [O.select(logits[t * E:(t + 1) * E], k) for t in range(batch)]
    ids = np.concatenate([s[0] for s in sel])
    w = np.concatenate([s[1] for s in sel])
    counts, _, _, _ = _check_group(O, ids, w, batch, k, E)
    assert counts[17] >= 128


def test_group_empty_and_all_skipped(O):
    counts, offsets, lst, active = O.group(np.array([1, 2], np.int32), np.array([0.0, -0.0], np.float32), 1, 2, 3)
    assert counts.tolist() == [0, 0, 0] and offsets.tolist() == [0, 0, 0, 0]
    assert lst.size == 0 and active.size == 0
