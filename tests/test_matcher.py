"""Token-range matcher and rolling hashes of the native library (host code,
no GPU calls) against the oracle: the reference's own cases
(tests/test_matcher.py:6-31), seeded random workloads on tiny vocabularies
where windows repeat and overlap, planted hash collisions, several scopes,
unregister / re-register order, and a long prompt with 256-token chunks.
Bit-exact: hashes and (start, segment) lists must be identical."""

import numpy as np
import pytest
import torch

import oracle as O
from cacheblend_vllm.hashing import content_hash, rolling_hash_values, rolling_hashes
from cacheblend_vllm.matcher import FingerprintRecord, TokenRangeMatcher
from cacheblend_vllm.types import SegmentId


def test_rolling_hash_matches_direct_hash_at_every_offset(golden):
    case = golden["rolling_hash_every_offset"]
    tokens, w = case["tokens"], case["window"]
    assert list(rolling_hashes(tokens, w)) == [
        (i, O.content_hash(tokens[i:i + w])) for i in range(len(tokens) - w + 1)
    ]
    assert rolling_hash_values(tokens, 8).shape == (0,)
    with pytest.raises(ValueError):
        rolling_hash_values(tokens, 0)


@pytest.mark.parametrize("window", [1, 2, 7, 256, 1000])
def test_rolling_hash_values_match_oracle(window):
    rng = np.random.default_rng(window)
    tokens = rng.integers(0, 152_000, size=4096)
    got = rolling_hash_values(tokens.tolist(), window)
    assert got.dtype == np.uint64
    np.testing.assert_array_equal(got, O.window_hashes(tokens, window))
    # every input form gives the same hashes
    np.testing.assert_array_equal(rolling_hash_values(tokens, window), got)
    np.testing.assert_array_equal(rolling_hash_values(torch.from_numpy(tokens), window), got)


def test_content_hash_matches_oracle_including_wrap():
    rng = np.random.default_rng(5)
    for n in (0, 1, 2, 3, 255, 256, 257):
        tokens = rng.integers(-1, 2**40, size=n).tolist()
        assert content_hash(tokens) == O.content_hash(tokens)


def test_matcher_finds_arbitrary_offsets_and_skips_overlaps(golden):
    case = golden["matcher_offsets_and_overlaps"]
    matcher = TokenRangeMatcher(chunk_size=case["chunk_size"])
    for scope, source, tokens in case["register"]:
        matcher.register(matcher.make_record(scope, source, tokens))
    matches = matcher.match("m", case["query"], start_offset=case["start_offset"])
    assert [[m.target_start, m.source_start] for m in matches] == case["expected_target_source"]
    assert matcher.match("other", case["query"]) == ()
    assert len(matcher) == 2


def test_hash_collision_is_verified_with_tokens(golden):
    case = golden["matcher_collision_verified"]
    matcher = TokenRangeMatcher(chunk_size=case["chunk_size"])
    fake = case["fake_record"]
    fake_id = SegmentId(fake["scope"], content_hash(fake["hash_of"]), fake["source_start"], 2)
    matcher.register(FingerprintRecord(fake_id, tuple(fake["tokens"])))
    assert list(matcher.match("m", case["query"])) == case["expected"]
    # a genuine record of the same hash, registered after the fake, matches
    real = matcher.make_record("m", 4, fake["hash_of"])
    matcher.register(real)
    (seg,) = matcher.match("m", case["query"])
    assert seg.segment_id == real.segment_id and seg.target_start == 0


def test_errors_and_argument_checks():
    with pytest.raises(ValueError, match="positive"):
        TokenRangeMatcher(0)
    matcher = TokenRangeMatcher(4)
    with pytest.raises(ValueError, match="exactly 4 tokens"):
        matcher.make_record("m", 0, [1, 2, 3])
    matcher.register(matcher.make_record("m", 0, [1, 2, 3, 4]))
    with pytest.raises(ValueError, match="outside"):
        matcher.match("m", [1, 2, 3, 4], start_offset=5)
    with pytest.raises(ValueError, match="outside"):
        matcher.match("m", [1, 2, 3, 4], start_offset=-1)
    assert matcher.match("m", [1, 2, 3, 4], start_offset=4) == ()
    assert matcher.match("m", []) == ()


def test_register_is_idempotent_and_unregister_removes():
    matcher = TokenRangeMatcher(2)
    rec = matcher.make_record("m", 0, [5, 6])
    matcher.register(rec)
    matcher.register(rec)
    assert len(matcher) == 1
    (seg,) = matcher.match("m", [0, 5, 6])
    assert matcher.validate([seg]) == (seg,)
    matcher.unregister(rec.segment_id)
    matcher.unregister(rec.segment_id)  # unknown ids are ignored
    assert len(matcher) == 0 and matcher.match("m", [0, 5, 6]) == ()
    assert matcher.validate([seg]) == ()


def _oracle_matches(records, scope, tokens, start, w):
    live = [(r.segment_id.model_scope, r.segment_id.content_hash, r.tokens) for r in records]
    return [(t, records[i].segment_id) for t, i in O.match_tokens(live, scope, tokens, start, w)]


@pytest.mark.parametrize("seed", range(12))
def test_random_workloads_match_oracle(seed):
    """Vocabulary of 3 tokens: windows repeat, overlap and collide in hash
    (fake ids planted with another chunk's hash). Registration order after
    unregister / re-register decides between equal-hash records, as in the
    reference."""
    rng = np.random.default_rng(seed)
    w = int(rng.integers(1, 5))
    matcher = TokenRangeMatcher(w)
    records = []  # registration order of live records
    for step in range(40):
        op = rng.random()
        scope = ("a", "b")[int(rng.integers(0, 2))]
        chunk = tuple(int(t) for t in rng.integers(0, 3, size=w))
        if op < 0.5:
            rec = matcher.make_record(scope, int(rng.integers(0, 64)), chunk)
        elif op < 0.7:  # fake id: another chunk's hash, these tokens
            other = tuple(int(t) for t in rng.integers(0, 3, size=w))
            rec = FingerprintRecord(SegmentId(scope, content_hash(other), int(rng.integers(0, 64)), w), chunk)
        elif records:
            victim = records[int(rng.integers(0, len(records)))]
            matcher.unregister(victim.segment_id)
            records.remove(victim)
            continue
        else:
            continue
        previous = next((r for r in records if r.segment_id == rec.segment_id), None)
        matcher.register(rec)
        if previous != rec:
            if previous is not None:
                records.remove(previous)
            records.append(rec)
        assert len(matcher) == len(records)
        tokens = rng.integers(0, 3, size=int(rng.integers(0, 40))).tolist()
        start = int(rng.integers(0, len(tokens) + 1))
        for s in ("a", "b", "c"):
            got = [(m.target_start, m.segment_id) for m in matcher.match(s, tokens, start)]
            assert got == _oracle_matches(records, s, tokens, start, w), (seed, step, s)


def test_long_prompt_with_planted_chunks_matches_oracle():
    """A 64K-token prompt over a real vocabulary with 256-token chunks copied
    in at arbitrary offsets (some overlapping, some truncated at the end)."""
    rng = np.random.default_rng(7)
    w = 256
    prompt = rng.integers(0, 152_000, size=65_536)
    matcher = TokenRangeMatcher(w)
    records = []
    for i in range(48):
        src = rng.integers(0, 152_000, size=w)
        rec = matcher.make_record("qwen", i * w, src.tolist())
        matcher.register(rec)
        records.append(rec)
        at = int(rng.integers(0, prompt.size - w // 2))
        take = min(w, prompt.size - at)
        prompt[at:at + take] = src[:take]
    for start in (0, 1, 4097):
        got = [(m.target_start, m.segment_id) for m in matcher.match("qwen", prompt, start)]
        want = _oracle_matches(records, "qwen", prompt.tolist(), start, w)
        assert got == want and len(got) > 10
