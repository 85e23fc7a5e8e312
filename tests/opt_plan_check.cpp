// Checks the optimizer update plan (plast_amd/csrc/opt_plan.hpp) on the CPU: piece splitting,
// workgroup numbering, launch grouping and the device-table cache, with host stand-ins for the
// device allocator and copy. Prints "ok" or the first rule broken, and exits non-zero on failure.
#include <cstdio>
#include <cstdlib>
#include <random>
#include <set>
#include <vector>

#include "opt_plan.hpp"

using plast::OptEntry;

static int g_fail = 0;

#define CHECK(cond)                                  \
  do {                                                \
    if (!(cond)) {                                    \
      std::printf("line %d: %s\n", __LINE__, #cond);  \
      g_fail = 1;                                     \
    }                                                 \
  } while (0)

static std::vector<OptEntry> with_counts(const std::vector<uint32_t> &counts) {
  std::vector<OptEntry> e;
  for (size_t i = 0; i < counts.size(); ++i) {
    OptEntry x{};
    x.n = i + 1;
    x.first_block = counts[i];
    e.push_back(x);
  }
  return e;
}

// Every entry in order, exactly once; each launch within the group and grid limits and holding
// the sum of its entries' workgroups.
static void check_groups(const std::vector<OptEntry> &e, size_t group, uint64_t max_blocks) {
  const auto g = plast::group_entries(e, group, max_blocks);
  size_t next = 0;
  for (const auto &l : g) {
    CHECK(l.first == next && l.count >= 1 && l.count <= group);
    uint64_t b = 0;
    for (size_t j = 0; j < l.count; ++j) b += e[l.first + j].first_block;
    CHECK(b == l.blocks && l.blocks <= max_blocks);
    next = l.first + l.count;
  }
  CHECK(next == e.size());
  // maximal: a launch ends only at the group size, at the grid limit, or at the last entry
  for (size_t i = 0; i + 1 < g.size(); ++i)
    CHECK(g[i].count == group || g[i].blocks + e[g[i].first + g[i].count].first_block > max_blocks);
}

int main() {
  // ---- add_tensor: pieces of at most max_piece elements, workgroup counts, offsets, null moments
  {
    std::vector<float> p(1000), g(1000), m(1000), v(1000);
    std::vector<OptEntry> e;
    plast::add_tensor(e, p.data(), g.data(), m.data(), v.data(), 0, true, 16, 64);
    CHECK(e.empty());
    plast::add_tensor(e, p.data(), g.data(), m.data(), v.data(), 64 * 2 + 15, true, 16, 64);
    CHECK(e.size() == 3);
    CHECK(e[0].n == 64 && e[1].n == 64 && e[2].n == 15);
    CHECK(e[0].first_block == 4 && e[1].first_block == 4 && e[2].first_block == 1);
    CHECK(e[1].p == p.data() + 64 && e[2].g == g.data() + 128 && e[2].m == m.data() + 128 &&
          e[2].v == v.data() + 128 && e[0].vec == 1);
    plast::add_tensor(e, p.data(), g.data(), nullptr, nullptr, 17, false, 16, 64);
    CHECK(e.size() == 4 && e[3].n == 17 && e[3].first_block == 2 && !e[3].m && !e[3].v &&
          e[3].vec == 0);
    CHECK(plast::total_blocks(e) == 11);
    plast::number_entries(e);
    CHECK(e[0].first_block == 0 && e[1].first_block == 4 && e[2].first_block == 8 &&
          e[3].first_block == 9);
  }

  // ---- group_entries: a worked case, then random ones
  {
    const auto e = with_counts({2, 2, 2, 1, 1, 1, 1});
    const auto g = plast::group_entries(e, 3, 5);
    CHECK(g.size() == 3);
    CHECK(g[0].first == 0 && g[0].count == 2 && g[0].blocks == 4);  // a third would pass 5
    CHECK(g[1].first == 2 && g[1].count == 3 && g[1].blocks == 4);  // the group size
    CHECK(g[2].first == 5 && g[2].count == 2 && g[2].blocks == 2);
    check_groups(e, 3, 5);
    CHECK(plast::group_entries({}, 3, 5).empty());
    std::mt19937 rng(7);
    for (int trial = 0; trial < 2000; ++trial) {
      const size_t n = rng() % 200;
      const uint64_t max_blocks = 1 + rng() % 100;
      const size_t group = 1 + rng() % 70;
      std::vector<uint32_t> c(n);
      for (auto &x : c) x = 1 + rng() % max_blocks;
      check_groups(with_counts(c), group, max_blocks);
    }
  }

  // ---- OptTableCache: reuse, replace, grow, failures
  {
    std::set<OptEntry *> live;
    int prepares = 0, allocs = 0, uploads = 0;
    bool fail_prepare = false, fail_alloc = false, fail_upload = false;
    auto prepare = [&]() {
      ++prepares;
      return !fail_prepare;
    };
    auto alloc = [&](size_t n) -> OptEntry * {
      ++allocs;
      if (fail_alloc) return nullptr;
      OptEntry *p = static_cast<OptEntry *>(std::calloc(n, sizeof(OptEntry)));
      live.insert(p);
      return p;
    };
    auto release = [&](OptEntry *p) {
      CHECK(live.count(p) == 1);
      live.erase(p);
      std::free(p);
    };
    std::vector<OptEntry> copied;
    auto upload = [&](OptEntry *dst, const std::vector<OptEntry> &src) {
      ++uploads;
      if (fail_upload) return false;
      CHECK(live.count(dst) == 1);
      for (size_t i = 0; i < src.size(); ++i) dst[i] = src[i];
      copied = src;
      return true;
    };
    auto same = [](const OptEntry *d, const std::vector<OptEntry> &e) {
      for (size_t i = 0; i < e.size(); ++i)
        if (d[i].n != e[i].n || d[i].first_block != e[i].first_block) return false;
      return true;
    };
    plast::OptTableCache c;
    const auto e1 = with_counts({1, 2, 3});
    const OptEntry *t1 = c.get(e1, prepare, alloc, release, upload);
    CHECK(t1 && same(t1, e1) && allocs == 1 && uploads == 1 && prepares == 1 && c.capacity() == 3);
    // an equal table: no wait, no upload
    CHECK(c.get(e1, prepare, alloc, release, upload) == t1 && uploads == 1 && prepares == 1);
    // the same size, other contents: uploaded into the same table after the wait
    const auto e2 = with_counts({1, 2, 4});
    CHECK(c.get(e2, prepare, alloc, release, upload) == t1 && uploads == 2 && prepares == 2 &&
          allocs == 1 && same(t1, e2));
    // larger: the old table released (after the wait), a new one allocated and filled
    const auto e3 = with_counts({1, 1, 1, 1, 1});
    const OptEntry *t3 = c.get(e3, prepare, alloc, release, upload);
    CHECK(t3 && allocs == 2 && live.size() == 1 && live.count(const_cast<OptEntry *>(t3)) == 1 &&
          c.capacity() == 5 && same(t3, e3));
    // smaller: reuses the larger table
    const auto e4 = with_counts({9});
    CHECK(c.get(e4, prepare, alloc, release, upload) == t3 && allocs == 2 && same(t3, e4));
    CHECK(c.get(e3, prepare, alloc, release, upload) == t3 && uploads == 5);
    // a failed upload returns null and the next call uploads again
    fail_upload = true;
    CHECK(c.get(e1, prepare, alloc, release, upload) == nullptr);
    fail_upload = false;
    const int before = uploads;
    CHECK(c.get(e1, prepare, alloc, release, upload) == t3 && uploads == before + 1 &&
          same(t3, e1));
    // ... and so does a failed wait, before anything is released or written
    fail_prepare = true;
    const int up = uploads, al = allocs;
    CHECK(c.get(e2, prepare, alloc, release, upload) == nullptr && uploads == up && allocs == al);
    fail_prepare = false;
    CHECK(c.get(e2, prepare, alloc, release, upload) == t3 && same(t3, e2));
    // a failed allocation leaves no table, and the next call allocates again
    fail_alloc = true;
    const auto e5 = with_counts({1, 1, 1, 1, 1, 1, 1, 1});
    CHECK(c.get(e5, prepare, alloc, release, upload) == nullptr && live.empty() &&
          c.capacity() == 0);
    fail_alloc = false;
    const OptEntry *t5 = c.get(e5, prepare, alloc, release, upload);
    CHECK(t5 && live.size() == 1 && c.capacity() == 8 && same(t5, e5));
    CHECK(c.get(e5, prepare, alloc, release, upload) == t5);
    for (OptEntry *p : live) std::free(p);  // the library keeps its table until the process ends
  }

  if (!g_fail) std::printf("ok\n");
  return g_fail;
}
