"""The logit-profile gate (rehip.qwen.logit_profile_check, after tests/qwen35_parity.rs:45-52)
on hand-made logits: it passes identical profiles and shifted ones (a constant offset leaves
every gap unchanged), fails a gap that moves by more than LOGIT_TOL, fails a flipped argmax only
where the reference's margin reaches TIE_FLOOR, and ignores tokens outside the reference's
top 5."""
import numpy as np

from rehip import qwen


def ref_logits():
    r = np.full(100, -10.0)
    r[[7, 3, 50, 9, 20]] = [5.0, 4.0, 3.5, 2.0, 1.0]     # top-5, margin 1.0 (decisive)
    return r


def test_identical_and_shifted_pass():
    r = ref_logits()
    assert qwen.logit_profile_check(r, r)["ok"]
    c = qwen.logit_profile_check(r, r + 123.0)
    assert c["ok"] and c["worst_gap_dev"] == 0.0 and c["decisive"]


def test_gap_beyond_tolerance_fails():
    r = ref_logits()
    g = r.copy()
    g[50] -= qwen.LOGIT_TOL + 0.05               # one top-5 gap moves by 0.8 nats
    c = qwen.logit_profile_check(r, g)
    assert not c["ok"] and abs(c["worst_gap_dev"] - (qwen.LOGIT_TOL + 0.05)) < 1e-12
    g = r.copy()
    g[50] -= qwen.LOGIT_TOL - 0.05               # within tolerance
    assert qwen.logit_profile_check(r, g)["ok"]


def test_argmax_flip_fails_only_when_decisive():
    r = ref_logits()
    g = r.copy()
    g[3] = 5.3                                   # got's argmax is token 3; gaps move by 0.3 / 1.3
    c = qwen.logit_profile_check(r, g, tol=2.0)
    assert c["decisive"] and not c["argmax_same"] and not c["ok"]
    r2 = r.copy()
    r2[3] = 4.7                                  # reference margin 0.3 < TIE_FLOOR: a tie
    g2 = r2.copy()
    g2[3], g2[7] = 5.0, 4.7                      # flipped argmax, gaps within 0.3
    c = qwen.logit_profile_check(r2, g2)
    assert not c["decisive"] and not c["argmax_same"] and c["ok"]


def test_tokens_outside_reference_top5_are_not_gated():
    r = ref_logits()
    g = r.copy()
    g[60] = 4.9                                  # a non-top-5 token jumps near the top
    assert qwen.logit_profile_check(r, g)["ok"]
