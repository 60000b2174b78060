// Slab sub-allocator behind hrt_alloc / hrt_free.
//
// Device memory is reserved from the driver in large slabs and carved into 512-byte aligned blocks,
// so that a training step's thousands of small tensors cost map lookups instead of driver calls.
// Semantics follow the reference runtime (vkrt/src/lib.rs:35-57, 645-839):
//   * block granularity / alignment 512 bytes; regular slabs of 512 MiB;
//   * requests >= 256 MiB get a dedicated slab that is returned to the driver when freed (after the
//     queued GPU work has drained, lib.rs:769-776);
//   * best fit over the free ranges, split on allocation, coalesced with both neighbours on free;
//   * an optional reservation cap (set_limit) shrinks slabs to cap/8 clamped to [64, 256] MiB with the
//     dedicated threshold at half a slab (lib.rs:1076-1091); near the cap a smaller slab that still
//     fits the request is made (lib.rs:717-728);
//   * when the driver (or the cap) refuses a slab, idle slabs are released and the reservation is
//     retried once (lib.rs:733-745);
//   * a transfer range must lie inside one live block's requested size (lib.rs:832-839).
// Differences by design: best fit is global over all slabs through a size index (O(log n) instead of
// a scan per slab), and free ranges never merge across slab boundaries even if two slabs happen to be
// adjacent in the address space.
//
// The class is independent of HIP: the device side is the `Backing` interface, so the host tests
// exercise it with a malloc-backed backing.
#pragma once

#include <cstdint>
#include <cstdio>
#include <iterator>
#include <map>
#include <set>
#include <string>
#include <utility>

namespace hrt {

struct Backing {
  virtual ~Backing() = default;
  // Reserve `size` bytes; on success store the base address and return true.
  virtual bool map(uint64_t size, uint64_t* base, std::string* err) = 0;
  // Release a reservation made by map().
  virtual void unmap(uint64_t base) = 0;
  // Wait for all queued device work (called before memory is returned to the driver).
  virtual void drain() = 0;
};

class SlabAllocator {
 public:
  static constexpr uint64_t kAlign = 512;
  static constexpr uint64_t kSlabBytes = 512ull << 20;
  static constexpr uint64_t kDedicatedMin = 256ull << 20;

  SlabAllocator(Backing* backing, uint64_t max_alloc) : backing_(backing), max_alloc_(max_alloc) { set_limit(0); }

  uint64_t max_alloc() const { return max_alloc_; }
  uint64_t live_bytes() const { return live_; }
  uint64_t peak_live_bytes() const { return peak_; }
  void reset_peak() { peak_ = live_; }
  size_t live_blocks() const { return blocks_.size(); }
  size_t slab_count() const { return slabs_.size(); }
  uint64_t limit() const { return limit_; }
  // While frozen, allocations are served from existing free ranges only (no driver calls at all).
  void set_frozen(bool f) { frozen_ = f; }

  uint64_t reserved_bytes() const {
    uint64_t r = 0;
    for (const auto& kv : slabs_) r += kv.second.size;
    return r;
  }

  void set_limit(uint64_t bytes) {
    limit_ = bytes;
    if (bytes > 0) {
      uint64_t s = bytes / 8;
      if (s > (256ull << 20)) s = 256ull << 20;
      if (s < (64ull << 20)) s = 64ull << 20;
      slab_bytes_ = s < max_alloc_ ? s : max_alloc_;
      dedicated_min_ = slab_bytes_ / 2;
    } else {
      slab_bytes_ = kSlabBytes < max_alloc_ ? kSlabBytes : max_alloc_;
      dedicated_min_ = kDedicatedMin < max_alloc_ / 2 ? kDedicatedMin : max_alloc_ / 2;
    }
    slab_bytes_ -= slab_bytes_ % kAlign;
  }

  // Returns the block address or 0 (with *err set).
  uint64_t alloc(uint64_t size, std::string* err) {
    if (size == 0) {
      *err = "allocation of size 0";
      return 0;
    }
    if (size > max_alloc_) {
      *err = "allocation of " + std::to_string(size) + " bytes exceeds the device limit of " + std::to_string(max_alloc_);
      return 0;
    }
    const uint64_t rounded = (size + kAlign - 1) / kAlign * kAlign;
    uint64_t addr = 0;
    if (frozen_) {
      addr = rounded < dedicated_min_ ? carve(rounded) : 0;
      if (addr == 0) {
        *err = "no free range of " + std::to_string(rounded) + " bytes and new device memory cannot be reserved now";
        return 0;
      }
    } else if (rounded >= dedicated_min_) {
      uint64_t base = 0;
      if (!new_slab_with_retry(rounded, /*dedicated=*/true, &base, err)) return 0;
      slabs_[base].used = rounded;
      addr = base;
    } else {
      addr = carve(rounded);
      if (addr == 0) {
        uint64_t want = slab_bytes_;
        if (limit_ > 0) {
          uint64_t res = reserved_bytes();
          uint64_t head = limit_ > res ? limit_ - res : 0;
          head -= head % kAlign;
          if (head >= rounded && head < want) want = head;
        }
        if (want < rounded) want = rounded;
        uint64_t base = 0;
        if (!new_slab_with_retry(want, /*dedicated=*/false, &base, err)) return 0;
        addr = carve(rounded);
        if (addr == 0) {
          *err = "allocation failed right after creating a slab";
          return 0;
        }
      }
    }
    auto slab_it = slab_of(addr);
    blocks_[addr] = Block{rounded, size, slab_it->first};
    live_ += rounded;
    if (live_ > peak_) peak_ = live_;
    return addr;
  }

  bool free(uint64_t addr, std::string* err) {
    auto it = blocks_.find(addr);
    if (it == blocks_.end()) {
      *err = "free of unknown address " + hex(addr);
      return false;
    }
    const Block blk = it->second;
    blocks_.erase(it);
    auto sit = slabs_.find(blk.slab);
    Slab& slab = sit->second;
    slab.used -= blk.size;
    live_ -= blk.size;
    if (slab.dedicated) {
      backing_->drain();  // queued kernels may still read it
      backing_->unmap(sit->first);
      slabs_.erase(sit);
      return true;
    }
    insert_free(blk.slab, addr, blk.size);
    return true;
  }

  // Return every slab without live blocks; returns how many were released.
  size_t empty_cache() {
    size_t n = 0;
    bool drained = false;
    for (auto it = slabs_.begin(); it != slabs_.end();) {
      if (it->second.used != 0) {
        ++it;
        continue;
      }
      if (!drained) {
        backing_->drain();
        drained = true;
      }
      if (!it->second.dedicated) {
        // an idle regular slab is exactly one free range
        auto f = free_.find(it->first);
        if (f != free_.end()) {
          by_size_.erase({f->second.len, f->first});
          free_.erase(f);
        }
      }
      backing_->unmap(it->first);
      it = slabs_.erase(it);
      ++n;
    }
    return n;
  }

  // True when addr is a live block carved from a regular (non-dedicated) slab.
  bool is_regular_block(uint64_t addr) const {
    auto it = blocks_.find(addr);
    if (it == blocks_.end()) return false;
    auto s = slabs_.find(it->second.slab);
    return s != slabs_.end() && !s->second.dedicated;
  }

  // True when [addr, addr + len) lies inside the requested size of one live block.
  // Size of the live block starting at base (0 if none).
  uint64_t block_bytes(uint64_t base) const {
    auto it = blocks_.find(base);
    return it == blocks_.end() ? 0 : it->second.size;
  }

  bool resolve(uint64_t addr, uint64_t len, std::string* err) const {
    auto it = blocks_.upper_bound(addr);
    if (it == blocks_.begin()) {
      *err = "unknown device address " + hex(addr);
      return false;
    }
    --it;
    const uint64_t base = it->first;
    const uint64_t end = base + it->second.req;
    if (addr >= end || len > end - addr) {
      if (addr >= base + it->second.size) {
        *err = "unknown device address " + hex(addr);
      } else {
        *err = "out-of-range access: addr=" + hex(addr) + " len=" + std::to_string(len) + " (block " + hex(base) +
               " of " + std::to_string(it->second.req) + " bytes)";
      }
      return false;
    }
    return true;
  }

 private:
  struct Slab {
    uint64_t size = 0;
    bool dedicated = false;
    uint64_t used = 0;
  };
  struct Block {
    uint64_t size;  // rounded
    uint64_t req;   // requested
    uint64_t slab;  // base of the owning slab
  };
  struct FreeRange {
    uint64_t len;
    uint64_t slab;
  };

  static std::string hex(uint64_t v) {
    char b[32];
    snprintf(b, sizeof(b), "0x%llx", (unsigned long long)v);
    return b;
  }

  std::map<uint64_t, Slab>::iterator slab_of(uint64_t addr) {
    auto it = slabs_.upper_bound(addr);
    --it;
    return it;
  }

  uint64_t carve(uint64_t rounded) {
    auto it = by_size_.lower_bound({rounded, 0});
    if (it == by_size_.end()) return 0;
    const uint64_t len = it->first, addr = it->second;
    by_size_.erase(it);
    auto f = free_.find(addr);
    const uint64_t slab = f->second.slab;
    free_.erase(f);
    if (len > rounded) {
      free_[addr + rounded] = FreeRange{len - rounded, slab};
      by_size_.insert({len - rounded, addr + rounded});
    }
    slabs_[slab].used += rounded;
    return addr;
  }

  void insert_free(uint64_t slab, uint64_t addr, uint64_t len) {
    auto next = free_.lower_bound(addr);
    if (next != free_.begin()) {
      auto prev = std::prev(next);
      if (prev->second.slab == slab && prev->first + prev->second.len == addr) {
        by_size_.erase({prev->second.len, prev->first});
        addr = prev->first;
        len += prev->second.len;
        free_.erase(prev);
      }
    }
    next = free_.lower_bound(addr + len);
    if (next != free_.end() && next->first == addr + len && next->second.slab == slab) {
      by_size_.erase({next->second.len, next->first});
      len += next->second.len;
      free_.erase(next);
    }
    free_[addr] = FreeRange{len, slab};
    by_size_.insert({len, addr});
  }

  bool new_slab_checked(uint64_t size, bool dedicated, uint64_t* base, std::string* err) {
    if (limit_ > 0) {
      uint64_t res = reserved_bytes();
      if (res + size > limit_) {
        *err = "memory limit of " + std::to_string(limit_ >> 20) + " MiB exceeded (reserved " + std::to_string(res >> 20) +
               " MiB + requested " + std::to_string(size >> 20) + " MiB)";
        return false;
      }
    }
    if (!backing_->map(size, base, err)) return false;
    Slab s;
    s.size = size;
    s.dedicated = dedicated;
    slabs_[*base] = s;
    if (!dedicated) {
      free_[*base] = FreeRange{size, *base};
      by_size_.insert({size, *base});
    }
    return true;
  }

  bool new_slab_with_retry(uint64_t size, bool dedicated, uint64_t* base, std::string* err) {
    if (new_slab_checked(size, dedicated, base, err)) return true;
    if (empty_cache() == 0) return false;
    std::string first = *err;
    if (new_slab_checked(size, dedicated, base, err)) return true;
    *err = first + " (still failing after releasing idle slabs; live " + std::to_string(live_) + " bytes)";
    return false;
  }

  Backing* backing_;
  uint64_t max_alloc_;
  uint64_t limit_ = 0;
  bool frozen_ = false;
  uint64_t slab_bytes_ = kSlabBytes;
  uint64_t dedicated_min_ = kDedicatedMin;
  uint64_t live_ = 0, peak_ = 0;
  std::map<uint64_t, Slab> slabs_;
  std::map<uint64_t, Block> blocks_;
  std::map<uint64_t, FreeRange> free_;
  std::set<std::pair<uint64_t, uint64_t>> by_size_;
};

}  // namespace hrt
