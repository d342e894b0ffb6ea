// Host-side driver for the token-range matcher's C ABI (token_matcher.hip)
// and the DMA run planner (cbk_memcpy_runs_commands, host_slab.hip), built
// with AddressSanitizer and UndefinedBehaviorSanitizer on the host pass
// by tests/test_host_sanitize.py. It runs seeded random sequences of
// register / re-register / unregister / match calls and compares every
// match with a brute-force model of the reference's matcher
// (cacheblend_vllm/matcher.py:53-126: leftmost non-overlapping windows whose
// hash is registered in the scope, the first record of that (scope, hash) in
// registration order whose tokens equal the window). Every output buffer is
// sized exactly, so a write past the matches found is an ASan report.
// A small vocabulary makes windows repeat; records registered under the hash
// of other tokens stand for hash collisions. Exit status 0 and a final "ok"
// line mean every check passed.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "cacheblend_hip.h"

namespace {

struct Rng {
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  int64_t below(int64_t n) { return int64_t(next() % uint64_t(n)); }
};

uint64_t window_hash(const int64_t* t, int64_t w) {
  uint64_t h = 0;
  for (int64_t j = 0; j < w; ++j) h = h * 1000003ull + (uint64_t(t[j]) + 1u);
  return h;
}

struct ModelRecord {
  uint64_t key, scope, hash, seq;
  std::vector<int64_t> tokens;
};

int failures = 0;
int64_t matches_checked = 0, match_calls = 0;

#define EXPECT(cond, ...)                      \
  do {                                         \
    if (!(cond)) {                             \
      std::fprintf(stderr, "FAIL: " __VA_ARGS__); \
      std::fprintf(stderr, "\n");              \
      if (++failures > 20) std::exit(1);       \
    }                                          \
  } while (0)

std::vector<int64_t> random_tokens(Rng& r, int64_t n, int64_t vocab) {
  std::vector<int64_t> t(static_cast<size_t>(n));
  for (auto& x : t) x = r.below(vocab) - (vocab > 3 ? 1 : 0);  // -1 appears as a token too
  return t;
}

void check_rolling(Rng& r) {
  for (int trial = 0; trial < 400; ++trial) {
    const int64_t w = 1 + r.below(40);
    const int64_t n = r.below(120);
    std::vector<int64_t> t = random_tokens(r, n, 1 + r.below(50000));
    const int64_t m = n >= w ? n - w + 1 : 0;
    std::vector<uint64_t> out(static_cast<size_t>(m));
    int rc = cbk_rolling_hashes(n ? t.data() : nullptr, n, w, m ? out.data() : nullptr);
    EXPECT(rc == CBK_OK, "rolling rc %d (n %lld w %lld)", rc, (long long)n, (long long)w);
    for (int64_t i = 0; i < m; ++i)
      EXPECT(out[size_t(i)] == window_hash(t.data() + i, w), "rolling hash %lld of n %lld w %lld",
             (long long)i, (long long)n, (long long)w);
  }
  EXPECT(cbk_rolling_hashes(nullptr, 5, 0, nullptr) == CBK_ERR_INVALID, "window 0 accepted");
  EXPECT(cbk_rolling_hashes(nullptr, -1, 3, nullptr) == CBK_ERR_INVALID, "negative n accepted");
}

std::vector<std::pair<int64_t, uint64_t>> model_match(const std::vector<ModelRecord>& recs,
                                                      uint64_t scope, const std::vector<int64_t>& t,
                                                      int64_t start, int64_t w) {
  std::vector<std::pair<int64_t, uint64_t>> out;
  const int64_t n = int64_t(t.size());
  int64_t next_allowed = start;
  for (int64_t target = start; target + w <= n; ++target) {
    if (target < next_allowed) continue;
    const uint64_t h = window_hash(t.data() + target, w);
    const ModelRecord* best = nullptr;
    for (const ModelRecord& rec : recs) {
      if (rec.scope != scope || rec.hash != h) continue;
      if (std::memcmp(rec.tokens.data(), t.data() + target, size_t(w) * sizeof(int64_t)) != 0) continue;
      if (best == nullptr || rec.seq < best->seq) best = &rec;
    }
    if (best != nullptr) {
      out.push_back({target, best->key});
      next_allowed = target + w;
    }
  }
  return out;
}

void run_sequence(uint64_t seed) {
  Rng r{seed};
  const int64_t widths[] = {1, 2, 3, 5, 8, 16};
  const int64_t w = widths[r.below(6)];
  const int64_t vocab = 2 + r.below(3);
  void* h = nullptr;
  EXPECT(cbk_matcher_create(w, &h) == CBK_OK && h != nullptr, "create");
  std::vector<ModelRecord> recs;
  uint64_t seq = 0;
  std::vector<int64_t> doc = random_tokens(r, 64 + r.below(200), vocab);
  for (int op = 0; op < 600; ++op) {
    const int kind = int(r.below(10));
    if (kind < 4) {  // register (a key may already be registered: replaced)
      ModelRecord rec;
      rec.key = uint64_t(r.below(40));
      rec.scope = uint64_t(r.below(3));
      if (r.below(3) == 0) {
        rec.tokens = random_tokens(r, w, vocab);
      } else {
        const int64_t at = r.below(int64_t(doc.size()) - w + 1);
        rec.tokens.assign(doc.begin() + at, doc.begin() + at + w);
      }
      rec.hash = window_hash(rec.tokens.data(), w);
      if (r.below(6) == 0) {  // a colliding record: the hash of other tokens
        std::vector<int64_t> other = random_tokens(r, w, vocab);
        rec.hash = window_hash(other.data(), w);
      }
      rec.seq = seq++;
      // A heap copy of exactly w tokens: the matcher must read no further.
      std::vector<int64_t> exact(rec.tokens);
      EXPECT(cbk_matcher_register(h, rec.scope, rec.key, rec.hash, exact.data()) == CBK_OK, "register");
      for (size_t i = 0; i < recs.size(); ++i)
        if (recs[i].key == rec.key) {
          recs.erase(recs.begin() + long(i));
          break;
        }
      recs.push_back(std::move(rec));
    } else if (kind < 6) {  // unregister, unknown keys included
      const uint64_t key = uint64_t(r.below(50));
      EXPECT(cbk_matcher_unregister(h, key) == CBK_OK, "unregister");
      for (size_t i = 0; i < recs.size(); ++i)
        if (recs[i].key == key) {
          recs.erase(recs.begin() + long(i));
          break;
        }
    } else {  // match a prompt: the document, a slice of it or fresh tokens
      std::vector<int64_t> t;
      if (kind == 9) {
        t = random_tokens(r, r.below(3 * w + 4), vocab);
      } else {
        const int64_t a = r.below(int64_t(doc.size()));
        const int64_t b = a + r.below(int64_t(doc.size()) - a + 1);
        t.assign(doc.begin() + a, doc.begin() + b);
      }
      const int64_t n = int64_t(t.size());
      const int64_t start = r.below(n + 1);
      const uint64_t scope = uint64_t(r.below(4));
      const auto want = model_match(recs, scope, t, start, w);
      const int64_t cap = int64_t(want.size());
      matches_checked += cap;
      ++match_calls;
      std::vector<int64_t> starts(static_cast<size_t>(cap));
      std::vector<uint64_t> keys(static_cast<size_t>(cap));
      // Exact-size token buffer: reading past the prompt is an ASan report.
      int64_t* tok = n ? new int64_t[size_t(n)] : nullptr;
      if (n) std::memcpy(tok, t.data(), size_t(n) * sizeof(int64_t));
      int64_t count = -1;
      int rc = cbk_matcher_match(h, scope, tok, n, start, cap ? starts.data() : nullptr,
                                 cap ? keys.data() : nullptr, cap, &count);
      EXPECT(rc == CBK_OK, "match rc %d: %s", rc, cbk_last_error());
      EXPECT(count == cap, "seed %llu op %d: %lld matches, model %lld", (unsigned long long)seed, op,
             (long long)count, (long long)cap);
      for (int64_t i = 0; i < cap && i < count; ++i)
        EXPECT(starts[size_t(i)] == want[size_t(i)].first && keys[size_t(i)] == want[size_t(i)].second,
               "seed %llu op %d match %lld", (unsigned long long)seed, op, (long long)i);
      if (cap > 0) {  // one slot too few: an error, not a write past the end
        std::vector<int64_t> s2(static_cast<size_t>(cap - 1));
        std::vector<uint64_t> k2(static_cast<size_t>(cap - 1));
        rc = cbk_matcher_match(h, scope, tok, n, start, cap > 1 ? s2.data() : nullptr,
                               cap > 1 ? k2.data() : nullptr, cap - 1, &count);
        EXPECT(rc == CBK_ERR_INVALID, "capacity %lld for %lld matches accepted", (long long)(cap - 1),
               (long long)cap);
      }
      rc = cbk_matcher_match(h, scope, tok, n, n + 1, nullptr, nullptr, 0, &count);
      EXPECT(rc == CBK_ERR_INVALID, "start past the end accepted");
      delete[] tok;
    }
    EXPECT(cbk_matcher_size(h) == int64_t(recs.size()), "size %lld, model %zu",
           (long long)cbk_matcher_size(h), recs.size());
  }
  EXPECT(cbk_matcher_destroy(h) == CBK_OK, "destroy");
}

// One writer registering and unregistering while readers match: the
// matcher's lock serialises them, and every match result must be one the
// model allows for some registration state (checked loosely: starts ascend,
// windows do not overlap, each key maps to a window equal to its record).
void run_concurrent(uint64_t seed) {
  const int64_t w = 4;
  void* h = nullptr;
  EXPECT(cbk_matcher_create(w, &h) == CBK_OK, "create");
  Rng r0{seed};
  std::vector<int64_t> doc = random_tokens(r0, 4096, 3);
  std::vector<std::vector<int64_t>> key_tokens(64);
  for (auto& kt : key_tokens) {
    const int64_t at = r0.below(int64_t(doc.size()) - w + 1);
    kt.assign(doc.begin() + at, doc.begin() + at + w);
  }
  std::thread writer([&] {
    Rng r{seed ^ 1};
    for (int i = 0; i < 4000; ++i) {
      const uint64_t key = uint64_t(r.below(64));
      if (r.below(3)) {
        const auto& kt = key_tokens[key];
        cbk_matcher_register(h, 0, key, window_hash(kt.data(), w), kt.data());
      } else {
        cbk_matcher_unregister(h, key);
      }
    }
  });
  std::vector<std::thread> readers;
  std::vector<int> bad(4, 0);
  for (int q = 0; q < 4; ++q)
    readers.emplace_back([&, q] {
      Rng r{seed + 7 * uint64_t(q) + 3};
      std::vector<int64_t> starts(doc.size());
      std::vector<uint64_t> keys(doc.size());
      for (int i = 0; i < 200; ++i) {
        const int64_t start = r.below(int64_t(doc.size()));
        int64_t count = 0;
        if (cbk_matcher_match(h, 0, doc.data(), int64_t(doc.size()), start, starts.data(), keys.data(),
                              int64_t(doc.size()), &count) != CBK_OK) {
          ++bad[size_t(q)];
          continue;
        }
        int64_t prev_end = start;
        for (int64_t k = 0; k < count; ++k) {
          const int64_t s = starts[size_t(k)];
          if (s < prev_end || keys[size_t(k)] >= 64 ||
              std::memcmp(doc.data() + s, key_tokens[keys[size_t(k)]].data(), size_t(w) * 8) != 0)
            ++bad[size_t(q)];
          prev_end = s + w;
        }
      }
    });
  writer.join();
  for (auto& t : readers) t.join();
  for (int q = 0; q < 4; ++q) EXPECT(bad[size_t(q)] == 0, "concurrent reader %d: %d bad results", q, bad[size_t(q)]);
  EXPECT(cbk_matcher_destroy(h) == CBK_OK, "destroy");
}

// The DMA planner of cbk_memcpy_runs (host_slab.hip) over exactly sized run
// tables mixing contiguous stretches, constant-pitch stretches, zero-byte runs
// and isolated runs: the command count lies between 1 and the number of
// non-empty runs, and a table built as one stretch folds into one command.
void check_copy_planner(Rng& r) {
  for (int trial = 0; trial < 3000; ++trial) {
    const int64_t n = 1 + r.below(48);
    std::vector<uint64_t> dst(static_cast<size_t>(n)), src(static_cast<size_t>(n)), bytes(static_cast<size_t>(n));
    const int shape = int(r.below(4));  // 0 contiguous, 1 pitched, 2 mixed, 3 isolated
    uint64_t d = 1 << 20, s = 1 << 30;
    const uint64_t w = 256 * uint64_t(1 + r.below(8));
    const uint64_t dp = w + 256 * uint64_t(r.below(4)), sp = w + 512 * uint64_t(r.below(4));
    int64_t nonzero = 0;
    for (int64_t i = 0; i < n; ++i) {
      uint64_t b = w;
      if (shape == 2 && r.below(4) == 0) b = r.below(2) ? 0 : 64 * uint64_t(1 + r.below(64));
      if (shape == 3) b = 64 * uint64_t(1 + r.below(64));
      dst[size_t(i)] = d;
      src[size_t(i)] = s;
      bytes[size_t(i)] = b;
      nonzero += b != 0;
      if (shape == 0) {
        d += b;
        s += b;
      } else if (shape == 1) {
        d += dp;
        s += sp;
      } else if (shape == 2) {
        d += r.below(2) ? b : dp + 4096 * uint64_t(r.below(3));
        s += r.below(2) ? b : sp;
      } else {
        d += b + 4096 * uint64_t(1 + r.below(1000));
        s -= 8192 * uint64_t(1 + r.below(100));
      }
    }
    int64_t commands = -1;
    EXPECT(cbk_memcpy_runs_commands(dst.data(), src.data(), bytes.data(), n, &commands) == CBK_OK,
           "planner rc");
    EXPECT(commands <= nonzero && (nonzero == 0 || commands >= 1), "%lld commands for %lld runs",
           (long long)commands, (long long)nonzero);
    if (shape == 0 || (shape == 1 && n > 1)) EXPECT(commands == 1, "one stretch gave %lld commands", (long long)commands);
  }
  int64_t commands = -1;
  EXPECT(cbk_memcpy_runs_commands(nullptr, nullptr, nullptr, 0, &commands) == CBK_OK && commands == 0, "empty table");
  EXPECT(cbk_memcpy_runs_commands(nullptr, nullptr, nullptr, -1, &commands) == CBK_ERR_INVALID, "negative count");
}

}  // namespace

int main() {
  Rng r{20261202};
  check_rolling(r);
  check_copy_planner(r);
  void* h = nullptr;
  EXPECT(cbk_matcher_create(0, &h) == CBK_ERR_INVALID, "chunk 0 accepted");
  EXPECT(cbk_matcher_create(4, nullptr) == CBK_ERR_INVALID, "NULL handle slot accepted");
  EXPECT(cbk_matcher_register(nullptr, 0, 0, 0, nullptr) == CBK_ERR_INVALID, "NULL matcher accepted");
  EXPECT(cbk_matcher_size(nullptr) == 0, "size of NULL");
  for (uint64_t seed = 1; seed <= 60; ++seed) run_sequence(seed);
  run_concurrent(99);
  if (failures) {
    std::fprintf(stderr, "%d failures\n", failures);
    return 1;
  }
  std::printf("ok: %lld matches over %lld match calls\n", (long long)matches_checked, (long long)match_calls);
  return 0;
}
