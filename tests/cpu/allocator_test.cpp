// Host test of the hrt slab sub-allocator with a fake backing (no GPU): the allocation semantics of the
// reference runtime's tests (vkrt/tests/basic.rs:78-182) plus the memory cap and the OOM retry.
#include <cassert>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "slab_allocator.h"

struct FakeBacking : hrt::Backing {
  uint64_t next = 0x100000000ull;
  uint64_t capacity = ~0ull;  // bytes the "driver" can hand out
  uint64_t mapped = 0;
  int drains = 0;
  std::map<uint64_t, uint64_t> live;
  bool map(uint64_t size, uint64_t* base, std::string* err) override {
    if (mapped + size > capacity) {
      *err = "fake out of memory";
      return false;
    }
    *base = next;
    next += (size + 0xFFFFF) / 0x100000 * 0x100000;  // the next slab may sit right after this one
    live[*base] = size;
    mapped += size;
    return true;
  }
  void unmap(uint64_t base) override {
    auto it = live.find(base);
    if (it == live.end()) {
      fprintf(stderr, "unmap of unknown base\n");
      std::abort();
    }
    mapped -= it->second;
    live.erase(it);
  }
  void drain() override { ++drains; }
};

#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      fprintf(stderr, "%s:%d CHECK failed: %s\n", __FILE__, __LINE__, #c); \
      return 1;                                                    \
    }                                                              \
  } while (0)

static int many_small_allocations() {
  FakeBacking fb;
  hrt::SlabAllocator a(&fb, 288ull << 30);
  std::string err;
  std::vector<uint64_t> addrs;
  for (int i = 0; i < 20000; ++i) addrs.push_back(a.alloc(1000 + (i % 7) * 100, &err));
  for (auto x : addrs) CHECK(x != 0 && x % 512 == 0);
  CHECK(a.slab_count() < 20);
  std::set<uint64_t> uniq(addrs.begin(), addrs.end());
  CHECK(uniq.size() == addrs.size());
  CHECK(a.live_blocks() == 20000);
  for (auto x : addrs) CHECK(a.free(x, &err));
  CHECK(a.live_bytes() == 0 && a.live_blocks() == 0);
  return 0;
}

static int coalescing_and_isolation() {
  FakeBacking fb;
  hrt::SlabAllocator a(&fb, 288ull << 30);
  std::string err;
  uint64_t x = a.alloc(4096, &err), y = a.alloc(4096, &err), z = a.alloc(4096, &err);
  CHECK(x && y && z);
  CHECK(a.free(y, &err));
  uint64_t big = a.alloc(8192, &err);
  CHECK(big != 0 && (big + 8192 <= x || big >= x + 4096) && (big + 8192 <= z || big >= z + 4096));
  const uint64_t reserved = a.reserved_bytes();
  CHECK(a.free(x, &err) && a.free(z, &err) && a.free(big, &err));
  uint64_t all = a.alloc(3 * 4096 + 8192, &err);
  CHECK(all != 0);
  CHECK(a.reserved_bytes() == reserved);  // served from the coalesced free range, no new slab
  CHECK(a.free(all, &err));
  // the whole slab is one free range again: an allocation of the full slab size fits without a new slab
  uint64_t whole = a.alloc(hrt::SlabAllocator::kDedicatedMin - 512, &err);
  CHECK(whole != 0 && a.slab_count() == 1);
  CHECK(a.free(whole, &err));
  return 0;
}

static int no_merge_across_adjacent_slabs() {
  FakeBacking fb;
  hrt::SlabAllocator a(&fb, 288ull << 30);
  std::string err;
  // fill slab 1 completely with two halves, force slab 2 (placed right after slab 1 by the fake backing)
  const uint64_t half = 128ull << 20;
  uint64_t p = a.alloc(half, &err), q = a.alloc(half, &err), r = a.alloc(half, &err), s = a.alloc(half, &err);
  CHECK(p && q && r && s && a.slab_count() == 1);
  uint64_t t = a.alloc(half, &err);
  CHECK(t && a.slab_count() == 2);
  CHECK(a.free(s, &err) && a.free(t, &err));
  // the tail of slab 1 and the head of slab 2 are adjacent addresses but must not form one range
  uint64_t big = a.alloc(200ull << 20, &err);
  CHECK(big != 0);
  CHECK(!(big < s + half && big + (200ull << 20) > s + half));
  return 0;
}

static int bounds_and_double_free() {
  FakeBacking fb;
  hrt::SlabAllocator a(&fb, 288ull << 30);
  std::string err;
  uint64_t x = a.alloc(64, &err);
  CHECK(x);
  CHECK(a.resolve(x, 64, &err));
  CHECK(a.resolve(x + 16, 48, &err));
  CHECK(!a.resolve(x, 128, &err));
  CHECK(err.find("out-of-range") != std::string::npos);
  CHECK(!a.resolve(0x1234, 4, &err));
  CHECK(!a.free(0x1234, &err));
  CHECK(a.free(x, &err));
  CHECK(!a.free(x, &err));
  CHECK(!a.resolve(x, 4, &err));
  CHECK(a.alloc(0, &err) == 0);
  CHECK(a.alloc((288ull << 30) + 1, &err) == 0);
  return 0;
}

static int dedicated_blocks_and_empty_cache() {
  FakeBacking fb;
  hrt::SlabAllocator a(&fb, 288ull << 30);
  std::string err;
  uint64_t big = a.alloc(300ull << 20, &err);
  CHECK(big);
  const uint64_t reserved = a.reserved_bytes();
  CHECK(reserved >= (300ull << 20));
  const int drains = fb.drains;
  CHECK(a.free(big, &err));
  CHECK(fb.drains == drains + 1);  // queued work drained before the memory goes back
  CHECK(a.reserved_bytes() < reserved);
  uint64_t small = a.alloc(1024, &err);
  CHECK(small && a.free(small, &err));
  CHECK(a.empty_cache() >= 1);
  CHECK(a.slab_count() == 0 && a.reserved_bytes() == 0 && fb.mapped == 0);
  return 0;
}

static int memory_limit_and_retry() {
  FakeBacking fb;
  hrt::SlabAllocator a(&fb, 288ull << 30);
  std::string err;
  a.set_limit(512ull << 20);  // slabs of 64 MiB, dedicated from 32 MiB
  std::vector<uint64_t> v;
  for (int i = 0; i < 7; ++i) v.push_back(a.alloc(60ull << 20, &err));
  for (auto x : v) CHECK(x);
  CHECK(a.reserved_bytes() <= (512ull << 20));
  CHECK(a.alloc(200ull << 20, &err) == 0);
  CHECK(err.find("memory limit") != std::string::npos);
  for (auto x : v) CHECK(a.free(x, &err));
  a.set_limit(0);
  // OOM retry: the driver holds 1 GiB; idle cached slabs are released and the reservation retried once
  FakeBacking fb2;
  fb2.capacity = 1ull << 30;
  hrt::SlabAllocator b(&fb2, 288ull << 30);
  uint64_t s1 = b.alloc(1024, &err);  // one 512 MiB slab
  CHECK(s1 && b.free(s1, &err));      // idle but cached
  uint64_t huge = b.alloc(768ull << 20, &err);  // needs the cached slab back
  CHECK(huge != 0);
  CHECK(b.free(huge, &err));
  uint64_t too_big = b.alloc(2ull << 30, &err);
  CHECK(too_big == 0);
  return 0;
}

static int peak_tracking() {
  FakeBacking fb;
  hrt::SlabAllocator a(&fb, 288ull << 30);
  std::string err;
  uint64_t x = a.alloc(1000, &err), y = a.alloc(3000, &err);
  CHECK(a.live_bytes() == 1024 + 3072);
  CHECK(a.free(y, &err));
  CHECK(a.peak_live_bytes() == 1024 + 3072);
  a.reset_peak();
  CHECK(a.peak_live_bytes() == 1024);
  CHECK(a.free(x, &err));
  return 0;
}

int main() {
  int (*tests[])() = {many_small_allocations, coalescing_and_isolation, no_merge_across_adjacent_slabs, bounds_and_double_free,
                      dedicated_blocks_and_empty_cache, memory_limit_and_retry, peak_tracking};
  int fails = 0;
  for (auto t : tests) fails += t();
  printf(fails ? "FAILED\n" : "ALL OK\n");
  return fails ? 1 : 0;
}
