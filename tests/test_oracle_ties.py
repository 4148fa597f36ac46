"""Tie rules and routing semantics of the CPU restatement, against closed
forms (no GPU):

- expert selection (qwen35_moe.hex:86-111): the rank of expert e is the
  number of experts with a larger router logit plus those with an equal
  logit and a lower index, so equal logits go to the lower index and the
  ids come out in descending logit order; the routing weights are the
  softmax over the selected logits only, its denominator summed in rank
  order (moe.hex:154-162);
- greedy argmax (fused_argmax.hex:2-47): the first index of the maximum,
  both when the maximum repeats inside one of the 256 contiguous chunks and
  when it repeats across chunks.

Each rule has a planted control in the restatement (oracle.planted): ties
toward the higher index, ascending selection, unnormalised weights, a
softmax over all experts, argmax toward the last index. Every control must
fail the same closed-form check."""
import numpy as np
import pytest

E, K = 256, 8


def closed_form_select(logits, k):
    """Stable descending rank: sort by (-logit, index)."""
    order = np.lexsort((np.arange(len(logits)), -logits.astype(np.float64)))
    ids = order[:k]
    sel = logits[ids].astype(np.float64)
    ex = np.exp(sel - sel[0])
    return ids, ex / ex.sum()


def tied_logits(rng, trials):
    """Router logits drawn from a few values, so that the top-k boundary and
    the ranks inside it are full of exact ties."""
    out = []
    for _ in range(trials):
        levels = rng.standard_normal(6).astype(np.float32)
        out.append(levels[rng.integers(0, 6, E)])
    return out


def select_mismatches(oracle, cases):
    bad_ids, worst_p = 0, 0.0
    for lg in cases:
        ids, probs = oracle.select(lg, K)
        want_ids, want_p = closed_form_select(lg, K)
        bad_ids += int(not np.array_equal(ids, want_ids))
        worst_p = max(worst_p, float(np.max(np.abs(probs.astype(np.float64) - want_p))))
    return bad_ids, worst_p


def test_selection_ties_go_to_the_lower_index(oracle):
    rng = np.random.default_rng(7)
    cases = tied_logits(rng, 64)
    # every case really has a tie among its selected experts
    for lg in cases:
        ids, _ = closed_form_select(lg, K)
        assert len(set(lg[ids].tolist())) < K
    bad, worst = select_mismatches(oracle, cases)
    assert bad == 0, f"{bad} of {len(cases)} selections differ from the stable rank"
    # routing weights: F32 exp (<= 1 ULP) and a serial F32 sum of 8 terms
    assert worst <= 2e-6, worst
    with oracle.planted("select_tie_high"):
        bad_high, _ = select_mismatches(oracle, cases)
    assert bad_high >= len(cases) // 2, f"tie-toward-higher control caught in only {bad_high} cases"


def test_selection_descending_and_normalised(oracle):
    rng = np.random.default_rng(8)
    cases = [(rng.standard_normal(E) * 3).astype(np.float32) for _ in range(32)]
    bad, worst = select_mismatches(oracle, cases)
    assert bad == 0 and worst <= 2e-6, (bad, worst)
    for lg in cases:
        _, probs = oracle.select(lg, K)
        assert abs(float(np.sum(probs.astype(np.float64))) - 1.0) <= 4e-7
    tol = 2e-6
    with oracle.planted("select_ascending"):
        bad_asc, _ = select_mismatches(oracle, cases)
    assert bad_asc == len(cases)
    for plant in ("prob_unnormalised", "softmax_all"):
        with oracle.planted(plant):
            _, miss = select_mismatches(oracle, cases)
        assert miss >= 3 * tol, f"{plant}: routing weights off by only {miss:.3g}"


def first_index_cases(oracle, vocab):
    """BF16 logits whose maximum repeats (i) inside one argmax chunk and
    (ii) across chunks, at chunk boundaries included."""
    rng = np.random.default_rng(9)
    chunk = (vocab + 255) // 256
    cases = []
    for where in ["inside", "across", "boundary", "everywhere"]:
        for _ in range(4):
            f = rng.standard_normal(vocab).astype(np.float32)
            top = np.float32(f.max() + 1.0)
            if where == "inside":
                c = int(rng.integers(0, 256)) * chunk
                pos = c + np.sort(rng.choice(min(chunk, vocab - c), 3, replace=False))
            elif where == "across":
                pos = np.sort(rng.choice(vocab, 5, replace=False))
            elif where == "boundary":
                c = int(rng.integers(1, 255)) * chunk
                pos = np.array([c - 1, c, c + chunk - 1])
            else:
                pos = np.arange(int(rng.integers(0, 97)), vocab, 97)
            f[pos] = top
            cases.append((oracle.bf16_round(f), int(pos.min())))
    return cases


@pytest.mark.parametrize("vocab", [4096, 248320, 1000])
def test_argmax_takes_the_first_index(oracle, vocab):
    cases = first_index_cases(oracle, vocab)
    for bits, first in cases:
        assert np.argmax(oracle.bf16_to_f32(bits)) == first  # the closed form
        assert oracle.argmax(bits) == first
    with oracle.planted("argmax_last"):
        missed = sum(oracle.argmax(bits) != first for bits, first in cases)
    assert missed == len(cases), f"last-index control caught in only {missed} of {len(cases)} cases"


def test_selection_with_nan_logits(oracle):
    """NaN logits under the reference's rank formula (qwen35_moe.hex:86-111):
    comparisons with NaN are false, so NaN counts among the lower indices of
    every expert (equal-or-unordered) and never as larger. For logits
    [3, NaN, 5, 1] the ranks are 1, 1, 1, 3 (worked by hand: e0 has e2
    above it; e1 has e0 below and unordered; e2 has e1 below and unordered;
    e3 has e0 and e2 above and e1 below and unordered). With k = 2: rank 0 is
    unassigned and keeps expert 0; rank 1 is shared by experts 0, 1 and 2
    and the largest index, 2, takes it (the ascending scatter). The weights
    are the softmax over the selected logits 3 and 5."""
    ids, probs = oracle.select(np.array([3.0, np.nan, 5.0, 1.0], dtype=np.float32), 2)
    assert ids.tolist() == [0, 2]
    e = np.exp(np.float64(2.0))
    assert abs(float(probs[0]) - 1.0 / (1.0 + e)) <= 2e-7
    assert abs(float(probs[1]) - e / (1.0 + e)) <= 2e-7
    # a NaN above every selected expert leaves the finite order untouched
    ids, _ = oracle.select(np.array([4.0, 2.0, 9.0, np.nan], dtype=np.float32), 2)
    assert ids.tolist() == [2, 0]
