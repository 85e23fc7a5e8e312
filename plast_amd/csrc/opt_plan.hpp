// opt_plan.hpp — the host-side plan of an optimizer update over a list of tensors: its entries (one
// per tensor, or per piece of a tensor longer than one launch's grid allows), their workgroup
// numbering, the launches of the kernel-argument path, and the cache of the device-resident entry
// table. Plain C++ (no HIP), so the rules can be checked on a machine without a GPU.
#pragma once

#include <cstdint>
#include <cstring>
#include <vector>

namespace plast {

// One tensor, or one piece of a tensor, of an update.
struct OptEntry {
  float *p;
  const float *g;
  float *m;
  float *v;
  uint64_t n;
  uint32_t first_block;  // its workgroup count until number_entries(), then its first workgroup
  uint32_t vec;          // 1: every pointer is 16-byte aligned
};
static_assert(sizeof(OptEntry) == 48, "no padding: entry tables are compared bytewise");

// Appends the entries of a tensor of n elements (m and v may be null): pieces of at most
// max_piece elements (a multiple of per_block), each holding its workgroup count, one workgroup
// per per_block elements.
inline void add_tensor(std::vector<OptEntry> &out, float *P, const float *G, float *M, float *V,
                       uint64_t n, bool aligned, uint64_t per_block, uint64_t max_piece) {
  for (uint64_t off = 0; off < n; off += max_piece) {
    const uint64_t len = n - off < max_piece ? n - off : max_piece;
    OptEntry e;
    e.p = P + off;
    e.g = G + off;
    e.m = M ? M + off : nullptr;
    e.v = V ? V + off : nullptr;
    e.n = len;
    e.first_block = uint32_t((len + per_block - 1) / per_block);
    e.vec = aligned ? 1u : 0u;
    out.push_back(e);
  }
}

// Total workgroups of the entries (which hold workgroup counts).
inline uint64_t total_blocks(const std::vector<OptEntry> &e) {
  uint64_t t = 0;
  for (const OptEntry &x : e) t += x.first_block;
  return t;
}

// Replaces each entry's workgroup count by its first workgroup number (the counts' prefix sum),
// for one launch over all of them; the caller checks that total_blocks() fits one grid.
inline void number_entries(std::vector<OptEntry> &e) {
  uint32_t blocks = 0;
  for (OptEntry &x : e) {
    const uint32_t need = x.first_block;
    x.first_block = blocks;
    blocks += need;
  }
}

// A launch of the kernel-argument path: entries [first, first + count) with `blocks` workgroups.
struct OptLaunch {
  size_t first;
  size_t count;
  uint64_t blocks;
};

// Consecutive runs of the entries (which hold workgroup counts), each of at most `group` entries
// whose workgroups fit a grid of max_blocks (every entry alone fits one).
inline std::vector<OptLaunch> group_entries(const std::vector<OptEntry> &e, size_t group,
                                            uint64_t max_blocks) {
  std::vector<OptLaunch> out;
  OptLaunch cur{0, 0, 0};
  for (size_t i = 0; i < e.size(); ++i) {
    const uint64_t need = e[i].first_block;
    if (cur.count && need > max_blocks - cur.blocks) {
      out.push_back(cur);
      cur = OptLaunch{i, 0, 0};
    }
    cur.count++;
    cur.blocks += need;
    if (cur.count == group) {
      out.push_back(cur);
      cur = OptLaunch{i + 1, 0, 0};
    }
  }
  if (cur.count) out.push_back(cur);
  return out;
}

// The device copy of the last entry table uploaded, and the host copy it was made from: a table
// equal to it is used as it is, another one is uploaded into it (after growing it if needed).
class OptTableCache {
 public:
  size_t capacity() const { return cap_; }

  // The device table holding e (null on failure, after which the next call uploads again).
  // prepare() (waits for earlier launches that may read the old table) runs before the old table
  // is released or overwritten; alloc(entries) returns a new table, release(ptr) frees one, and
  // upload(ptr, e) copies e into it; each returns false or null on failure.
  template <class Prepare, class Alloc, class Release, class Upload>
  const OptEntry *get(const std::vector<OptEntry> &e, Prepare prepare, Alloc alloc,
                      Release release, Upload upload) {
    if (dev_ && e.size() == host_.size() &&
        std::memcmp(e.data(), host_.data(), e.size() * sizeof(OptEntry)) == 0)
      return dev_;
    host_.clear();  // until the upload below succeeds
    if (!prepare()) return nullptr;
    if (e.size() > cap_) {
      if (dev_) release(dev_);
      dev_ = nullptr;
      cap_ = 0;
      dev_ = alloc(e.size());
      if (!dev_) return nullptr;
      cap_ = e.size();
    }
    if (!upload(dev_, e)) return nullptr;
    host_ = e;
    return dev_;
  }

 private:
  std::vector<OptEntry> host_;
  OptEntry *dev_ = nullptr;
  size_t cap_ = 0;
};

}  // namespace plast
