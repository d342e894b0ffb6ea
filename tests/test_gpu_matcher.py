"""The token-range matcher's native-vs-oracle checks, run again under the
``gpu`` marker so the library loaded on an MI355X machine (the same
libcacheblend_hip.so whose host part holds ``cbk_matcher_*`` and
``cbk_rolling_hashes``) is the one checked there. The matcher is host code;
the checks are those of test_matcher.py (reference hashing.py:18-53,
matcher.py:80-125)."""

import pytest

from test_matcher import (  # noqa: F401 - collected again under this module's marker
    test_content_hash_matches_oracle_including_wrap,
    test_hash_collision_is_verified_with_tokens,
    test_long_prompt_with_planted_chunks_matches_oracle,
    test_matcher_finds_arbitrary_offsets_and_skips_overlaps,
    test_random_workloads_match_oracle,
    test_rolling_hash_matches_direct_hash_at_every_offset,
    test_rolling_hash_values_match_oracle,
)

pytestmark = pytest.mark.gpu
