"""Pins the window-driver restatement (oracle/transcribe_ref.py and the C
process_logits / compute_logprobs of oracle/refcpu.c) with the reference's own
unit cases for those functions (decode.rs:4890-5811, restated here on the same
synthetic English-only tokenizer: 51864 tokens, eot 50256, timestamp_begin
50363, " " at id 1), plus closed forms of the log-softmax."""
import math

import numpy as np
import pytest

from franken_whisper_amd import abi
from oracle import oracle as O
from oracle import transcribe_ref as R

V = 51864
EOT, SOT, TRANSLATE, TRANSCRIBE, SOLM, PREV, NOSP, NOTS, BEG = 50256, 50257, 50357, 50358, 50359, 50360, 50361, 50362, 50363
CHUNK = 3000


def filt():
    return abi.Filter(EOT, SOT, PREV, SOLM, NOSP, NOTS, TRANSLATE, TRANSCRIBE, BEG, 1, 100)


def cfg(no_ts=False, mit=-1, max_tokens=-1, blank=True):
    return O.RefFilterCfg(1 if blank else 0, 1 if no_ts else 0, mit, max_tokens)


def pl(logits, prev, has_ts, delta, n=None, c=None):
    out, lp, forced = O.process_logits(filt(), c or cfg(), np.asarray(logits, np.float32), prev, has_ts, delta,
                                       len(prev) if n is None else n)
    return out, lp


def supp(x, i):
    return x[i] == -np.inf


def zeros():
    return np.zeros(V, np.float32)


def text_dominant():
    v = np.full(V, -30.0, np.float32)
    v[:EOT] = 5.0
    return v


def test_blank_and_eot_suppressed_at_step0():
    out, _ = pl(zeros(), [], False, CHUNK)
    assert supp(out, EOT) and supp(out, 1)
    out, _ = pl(text_dominant(), [2], False, CHUNK)
    assert not supp(out, EOT) and not supp(out, 1)


def test_control_tokens_always_suppressed():
    out, _ = pl(zeros(), [2], False, CHUNK)
    for i in (SOT, NOSP, SOLM, PREV, NOTS, TRANSLATE, TRANSCRIBE):
        assert supp(out, i), i


def test_timestamp_pairing_two_ts_back_to_back_forbids_timestamp():
    out, _ = pl(zeros(), [BEG + 5, BEG + 10], True, 20)
    assert supp(out, BEG + 50) and not supp(out, 2)


def test_timestamp_pairing_one_ts_open_forces_timestamp_or_eot():
    lg = np.full(V, -5.0, np.float32)
    lg[EOT] = 20.0
    out, _ = pl(lg, [2, BEG + 10], True, 20)
    assert supp(out, 2) and not supp(out, EOT)


def test_timestamp_monotonicity_masks_earlier_timestamps():
    out, _ = pl(zeros(), [2], True, 100)
    assert supp(out, BEG + 10) and not supp(out, BEG + 60)


def test_max_initial_ts_clamps_first_step():
    out, _ = pl(zeros(), [], False, CHUNK, c=cfg(mit=50))
    assert supp(out, BEG + 51) and not supp(out, BEG + 50)
    assert R.max_initial_tid(1500) == 50


def test_logsumexp_forces_timestamp_when_ts_mass_exceeds_text():
    lg = np.full(V, -10.0, np.float32)
    lg[2] = 1.0
    lg[BEG:BEG + 200] = 0.5
    out, _ = pl(lg, [2], False, 0)
    assert supp(out, 2) and supp(out, 0) and not supp(out, BEG + 1)


def test_logsumexp_keeps_text_when_text_dominates():
    lg = np.full(V, -20.0, np.float32)
    lg[2] = 10.0
    lg[BEG:BEG + 3] = -5.0
    out, lp = pl(lg, [2], False, 0)
    assert not supp(out, 2) and O.argmax_first(out) == 2


def test_no_timestamps_mode_masks_all_timestamps():
    out, _ = pl(zeros(), [2], False, CHUNK, c=cfg(no_ts=True))
    assert supp(out, BEG) and supp(out, BEG + 100) and not supp(out, 2)


def test_user_budget_filter_fires_at_loop_boundary():
    lg = np.full(V, -20.0, np.float32)
    lg[5] = 10.0
    c = cfg(max_tokens=3, blank=False)
    out, _ = pl(lg, [], False, 0, n=2, c=c)
    assert not supp(out, 5)
    out, _ = pl(lg, [], False, 0, n=3, c=c)
    assert supp(out, 5)


def test_max_tokens_filter_inert_in_no_timestamps_mode_and_off_when_none():
    out, _ = pl(text_dominant(), [2], False, CHUNK, n=5, c=cfg(no_ts=True, max_tokens=2))
    assert not supp(out, 2)
    out, _ = pl(text_dominant(), [2], False, CHUNK, n=99, c=cfg(max_tokens=-1))
    assert not supp(out, 2)
    out, _ = pl(text_dominant(), [2], False, CHUNK, n=4, c=cfg(max_tokens=4))
    assert supp(out, 2) and supp(out, 0) and not supp(out, BEG + 1)


def test_single_timestamp_ending_matches_upstream_semantics():
    beg = 100
    assert not R.single_timestamp_ending([5, beg + 10, 50], beg, True, None)
    assert R.single_timestamp_ending([5, beg + 10], beg, True, None)
    assert not R.single_timestamp_ending([5, beg + 10], beg, True, 1)
    assert R.single_timestamp_ending([5, beg + 10], beg, True, 2)
    assert R.single_timestamp_ending([5, beg + 10], beg, False, 1)
    assert not R.single_timestamp_ending([beg + 10], beg, True, None)
    assert not R.single_timestamp_ending([], beg, True, None)


def test_unclosed_window_rescue_requires_no_prior_output():
    assert R.should_rescue_unclosed_window(0, True, False)
    assert R.should_rescue_unclosed_window(3000, True, False)
    assert not R.should_rescue_unclosed_window(2800, True, True)
    assert not R.should_rescue_unclosed_window(0, False, False)


def test_short_tail_prompt_clearing_predicate():
    assert not R.should_clear_short_tail_prompt(0, 1000)
    assert R.should_clear_short_tail_prompt(600, 1000)
    assert R.should_clear_short_tail_prompt(500, 1000)
    assert not R.should_clear_short_tail_prompt(400, 1000)


# build_segments (decode.rs:5606-5790) on the synthetic tokenizer's vocab
VOCAB = [b"."] * EOT
VOCAB[1], VOCAB[2], VOCAB[3] = b" ", b"hello", b" world"


def segs(tokens, plogs, seek, delta, end, split):
    return R.build_segments(VOCAB, tokens, plogs, seek, delta, end, split, BEG, EOT)


def test_segments_from_timestamp_pairs_and_confidence():
    s = segs([BEG, 2, 3, BEG + 150], [-0.1] * 4, 0, 3000, 10 ** 12, True)
    assert len(s) == 1 and s[0][:3] == (0, 300, "hello world") and s[0][3] > 0
    s = segs([BEG, 2, 3, BEG + 150], [-5.0, 0.0, 0.0, -5.0], 0, 3000, 10 ** 12, True)
    assert abs(s[0][3] - 1.0) < 1e-9
    assert R.text_confidence([BEG, BEG + 10], [-0.1, -0.1], BEG, EOT) is None
    assert R.text_confidence([2, 3], [0.0, float("nan")], BEG, EOT) == 1.0
    assert R.text_confidence([2, 3], [float("nan"), float("inf")], BEG, EOT) is None


def test_segments_two_pairs_open_tail_single_offset_clamped():
    s = segs([BEG, 2, BEG + 50, 3, BEG + 100], [-0.2] * 5, 0, 2000, 10 ** 12, True)
    assert [x[:3] for x in s] == [(0, 100, "hello"), (100, 200, "world")]
    s = segs([BEG, 2, BEG + 50, 3], [-0.2] * 4, 0, 1500, 10 ** 12, True)
    assert s[1][:3] == (100, 1500, "world")
    s = segs([2, 3], [-0.3] * 2, 500, 3000, 10 ** 12, False)
    assert s[0][:3] == (500, 3500, "hello world")
    s = segs([BEG, 2, BEG + 50], [-0.1] * 3, 3000, 3000, 10 ** 12, True)
    assert s[0][:2] == (3000, 3100)
    s = segs([BEG, 2, 3, BEG + 500], [-0.1] * 4, 0, 3000, 600, True)
    assert s[0][:3] == (0, 600, "hello world")
    s = segs([BEG, 2, BEG + 200, 3], [-0.1] * 4, 0, 3000, 600, True)
    assert len(s) == 2 and s[1][1] == 600


def test_carried_prompt_and_split_prompt():
    assert R.carried_prompt_tokens(PREV, [], [1, 2, 3, 4], 3) == [PREV, 3, 4]
    assert R.carried_prompt_tokens(PREV, [9], [1, 2, 3, 4], 4) == [PREV, 9, 3, 4]
    assert R.split_carried_prompt([1, 2, 3, 4, 5], True, 4) == ([3, 4, 5], [])
    assert R.split_carried_prompt([1, 2, 3], False, 4) == ([], [1, 2, 3])
    assert R.seek_end_cs(0) == 10 and R.seek_end_cs(16000) == 1 + (16000 - 200) // 160


def test_compute_logprobs_closed_forms_and_non_finite_lanes():
    x = np.array([np.inf, 0.0, -1.0], np.float32)
    lp = O.compute_logprobs(x)
    assert lp[0] == -np.inf and np.isfinite(lp[1]) and np.isfinite(lp[2])
    lp = O.compute_logprobs(np.array([np.nan, 0.0, -1.0], np.float32))
    assert lp[0] == -np.inf and np.isfinite(lp[1:]).all()
    # uniform row: every lane log(1/n); two lanes a, b: log-sigmoid
    lp = O.compute_logprobs(np.zeros(8, np.float32))
    assert np.allclose(lp, math.log(1 / 8), atol=1e-6)
    lp = O.compute_logprobs(np.array([2.0, -1.0], np.float32))
    assert abs(lp[0] - (-math.log1p(math.exp(-3.0)))) < 1e-6
    assert O.compute_logprobs(np.full(4, -np.inf, np.float32)).tolist() == [-np.inf] * 4


def test_rust_trim_and_lossy_text():
    v = [b" \x85"[0:1], b"\xe2\x80\x83", b"\xff", b"a", b"\xc3", b"\xa9"]
    # ' ' + EM SPACE trimmed; a lone 0xff is U+FFFD; c3 a9 joins to e-acute
    assert R.decode_text(v, [0, 1, 3, 4, 5, 0], 6) == "aé"
    assert R.decode_text(v, [2, 3], 6) == "�a"
