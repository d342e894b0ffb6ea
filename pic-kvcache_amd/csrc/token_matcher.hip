// Token-range matcher for the blend lookup: finds stored 256-token chunks at
// any offset of a prompt (the reference's TokenRangeMatcher and rolling
// hash, cacheblend_vllm/matcher.py:22-131, hashing.py:10-53), host code.
//
// A chunk's identity hash is the polynomial hash of its tokens,
//   H(t_0..t_{w-1}) = sum_j (t_j + 1) * B^(w-1-j)  (mod 2^64), B = 1,000,003,
// so the hash of every window of a prompt follows from its predecessor in
// O(1): H(i+1) = (H(i) - (t_i + 1) * B^(w-1)) * B + (t_{i+w} + 1). The
// reference evaluates each window independently (an O(n * w) matrix product).
// Matching rolls the window hash left to right, tests it against a 64 Kibit
// filter of the scope's registered hashes (indexed by the hash's top 16
// bits, which depend on every token; 8 KiB, cache resident) and only on a
// filter hit looks it up exactly, verifies the tokens, and keeps the
// leftmost non-overlapping matches.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "cbk_common.hpp"

namespace {

constexpr uint64_t kBase = 1000003ull;

struct Record {
  uint64_t key;
  std::vector<int64_t> tokens;
};

struct PairHash {
  size_t operator()(const std::pair<uint64_t, uint64_t>& p) const noexcept {
    return std::hash<uint64_t>()(p.first * 0x9e3779b97f4a7c15ull ^ p.second);
  }
};

constexpr int kFilterBits = 16;
constexpr size_t kFilterWords = (size_t(1) << kFilterBits) / 64;

inline uint32_t filter_slot(uint64_t h) { return uint32_t(h >> (64 - kFilterBits)); }

struct Scope {
  std::unordered_set<uint64_t> hashes;
  std::vector<uint64_t> filter = std::vector<uint64_t>(kFilterWords, 0);
  bool stale = false;  // a hash was removed: rebuild the filter before use

  void add(uint64_t h) {
    hashes.insert(h);
    filter[filter_slot(h) >> 6] |= uint64_t(1) << (filter_slot(h) & 63);
  }
  void rebuild() {
    std::fill(filter.begin(), filter.end(), 0);
    for (uint64_t h : hashes) filter[filter_slot(h) >> 6] |= uint64_t(1) << (filter_slot(h) & 63);
    stale = false;
  }
  bool maybe(uint64_t h) const { return (filter[filter_slot(h) >> 6] >> (filter_slot(h) & 63)) & 1; }
};

struct Matcher {
  std::mutex mu;
  int64_t chunk = 0;
  std::unordered_map<std::pair<uint64_t, uint64_t>, std::vector<Record>, PairHash> by_scope_hash;
  std::unordered_map<uint64_t, Scope> scope_hashes;
  std::unordered_map<uint64_t, std::pair<uint64_t, uint64_t>> by_key;  // key -> (scope, hash)
};

uint64_t power(uint64_t base, int64_t e) {
  uint64_t r = 1;
  while (e > 0) {
    if (e & 1) r *= base;
    base *= base;
    e >>= 1;
  }
  return r;
}

void rolling(const int64_t* tokens, int64_t n, int64_t w, uint64_t* out) {
  const uint64_t top = power(kBase, w - 1);
  uint64_t h = 0;
  for (int64_t j = 0; j < w; ++j) h = h * kBase + (uint64_t(tokens[j]) + 1u);
  out[0] = h;
  for (int64_t i = 1; i + w <= n; ++i) {
    h = (h - (uint64_t(tokens[i - 1]) + 1u) * top) * kBase + (uint64_t(tokens[i + w - 1]) + 1u);
    out[i] = h;
  }
}

void unregister_locked(Matcher* m, uint64_t key) {
  auto it = m->by_key.find(key);
  if (it == m->by_key.end()) return;
  const auto sh = it->second;
  m->by_key.erase(it);
  auto rec = m->by_scope_hash.find(sh);
  if (rec == m->by_scope_hash.end()) return;
  auto& v = rec->second;
  v.erase(std::remove_if(v.begin(), v.end(), [key](const Record& r) { return r.key == key; }), v.end());
  if (v.empty()) {
    m->by_scope_hash.erase(rec);
    auto sc = m->scope_hashes.find(sh.first);
    if (sc != m->scope_hashes.end()) {
      sc->second.hashes.erase(sh.second);
      sc->second.stale = true;
      if (sc->second.hashes.empty()) m->scope_hashes.erase(sc);
    }
  }
}

}  // namespace

extern "C" {

int cbk_rolling_hashes(const int64_t* tokens, int64_t n, int64_t window, uint64_t* out) {
  cbk::clear_error();
  CBK_REQUIRE(window > 0, "window must be positive");
  CBK_REQUIRE(n >= 0, "negative token count");
  if (n < window) return CBK_OK;
  CBK_REQUIRE(tokens != nullptr && out != nullptr, "NULL pointer");
  rolling(tokens, n, window, out);
  return CBK_OK;
}

int cbk_matcher_create(int64_t chunk_size, void** out_handle) {
  cbk::clear_error();
  CBK_REQUIRE(out_handle != nullptr, "out_handle is NULL");
  CBK_REQUIRE(chunk_size > 0, "chunk_size must be positive");
  Matcher* m = new Matcher;
  m->chunk = chunk_size;
  *out_handle = m;
  return CBK_OK;
}

int cbk_matcher_destroy(void* handle) {
  cbk::clear_error();
  delete static_cast<Matcher*>(handle);
  return CBK_OK;
}

int cbk_matcher_register(void* handle, uint64_t scope, uint64_t key, uint64_t hash, const int64_t* tokens) {
  cbk::clear_error();
  CBK_REQUIRE(handle != nullptr && tokens != nullptr, "NULL argument");
  Matcher* m = static_cast<Matcher*>(handle);
  std::lock_guard<std::mutex> lock(m->mu);
  unregister_locked(m, key);  // re-registering a key replaces its record
  Record r;
  r.key = key;
  r.tokens.assign(tokens, tokens + m->chunk);
  m->by_scope_hash[{scope, hash}].push_back(std::move(r));
  m->scope_hashes[scope].add(hash);
  m->by_key[key] = {scope, hash};
  return CBK_OK;
}

int cbk_matcher_unregister(void* handle, uint64_t key) {
  cbk::clear_error();
  CBK_REQUIRE(handle != nullptr, "NULL handle");
  Matcher* m = static_cast<Matcher*>(handle);
  std::lock_guard<std::mutex> lock(m->mu);
  unregister_locked(m, key);
  return CBK_OK;
}

int64_t cbk_matcher_size(void* handle) {
  if (handle == nullptr) return 0;
  Matcher* m = static_cast<Matcher*>(handle);
  std::lock_guard<std::mutex> lock(m->mu);
  return int64_t(m->by_key.size());
}

int cbk_matcher_match(void* handle, uint64_t scope, const int64_t* tokens, int64_t n, int64_t start,
                      int64_t* out_starts, uint64_t* out_keys, int64_t capacity, int64_t* out_count) {
  cbk::clear_error();
  CBK_REQUIRE(handle != nullptr && out_count != nullptr, "NULL argument");
  CBK_REQUIRE(start >= 0 && start <= n, "start_offset is outside the token sequence");
  Matcher* m = static_cast<Matcher*>(handle);
  *out_count = 0;
  const int64_t w = m->chunk;
  std::lock_guard<std::mutex> lock(m->mu);
  auto sc = m->scope_hashes.find(scope);
  if (sc == m->scope_hashes.end() || n - start < w) return CBK_OK;
  CBK_REQUIRE(tokens != nullptr, "tokens is NULL");
  Scope& known = sc->second;
  if (known.stale) known.rebuild();
  const uint64_t top = power(kBase, w - 1);
  const int64_t* t = tokens;
  uint64_t h = 0;
  for (int64_t j = start; j < start + w; ++j) h = h * kBase + (uint64_t(t[j]) + 1u);
  int64_t count = 0, next_allowed = start;
  for (int64_t target = start;; ++target) {
    // h is the hash of t[target .. target + w)
    if (target >= next_allowed && known.maybe(h) && known.hashes.count(h)) {
      auto rec = m->by_scope_hash.find({scope, h});
      if (rec != m->by_scope_hash.end()) {
        for (const Record& r : rec->second) {
          if (std::memcmp(r.tokens.data(), t + target, size_t(w) * sizeof(int64_t)) != 0) continue;
          CBK_REQUIRE(count < capacity, "more than %lld matches", (long long)capacity);
          out_starts[count] = target;
          out_keys[count] = r.key;
          ++count;
          next_allowed = target + w;
          break;
        }
      }
    }
    if (target + w >= n) break;
    h = (h - (uint64_t(t[target]) + 1u) * top) * kBase + (uint64_t(t[target + w]) + 1u);
  }
  *out_count = count;
  return CBK_OK;
}

}  // extern "C"
