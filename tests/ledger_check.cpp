// Checks the workspace ledger's rules (plast_amd/csrc/ws_ledger.hpp) with counting stand-ins for
// the device allocator: prints "ok" or the first rule broken, and exits non-zero on failure.
#include <cstdio>
#include <cstdlib>
#include <set>

#include "ws_ledger.hpp"

static std::set<void *> g_live;  // buffers allocated and not yet released
static int g_fail = 0;

#define CHECK(cond)                                               \
  do {                                                            \
    if (!(cond)) {                                                \
      std::printf("line %d: %s\n", __LINE__, #cond);              \
      g_fail = 1;                                                 \
    }                                                             \
  } while (0)

int main() {
  auto alloc = [](size_t n) -> void * {
    void *p = std::malloc(n);
    g_live.insert(p);
    return p;
  };
  auto release = [](void *p) {
    CHECK(g_live.count(p) == 1);  // never released twice, never an unknown buffer
    g_live.erase(p);
    std::free(p);
  };
  auto fail = [](size_t) -> void * { return nullptr; };
  plast::WorkspaceLedger<3> w;
  int g1 = 0, g2 = 0, g3 = 0;  // stand-in graph handles

  // no graph alive: an outgrown buffer is released at once, a fitting request keeps the buffer
  void *a = w.grow(0, 100, 128, alloc, release);
  CHECK(a && w.bytes(0) == 128 && g_live.size() == 1);
  CHECK(w.grow(0, 128, 128, alloc, release) == a);
  void *b = w.grow(0, 129, 256, alloc, release);
  CHECK(b && b != a && g_live.size() == 1 && w.retired() == 0);

  // two graphs alive: outgrown buffers are retired, not released, through several growths
  w.graph_created(&g1);
  w.graph_created(&g2);
  void *c = w.grow(0, 300, 512, alloc, release);
  CHECK(c && g_live.count(b) == 1 && w.retired() == 1);
  void *d = w.grow(0, 600, 1024, alloc, release);
  CHECK(d && g_live.count(c) == 1 && w.retired() == 2);
  void *e = w.grow(1, 10, 64, alloc, release);  // a first buffer retires nothing
  CHECK(e && w.retired() == 2);

  // an unknown graph changes nothing; the first of two graphs destroyed keeps the retired buffers
  CHECK(!w.graph_destroyed(&g3, release));
  CHECK(w.graph_destroyed(&g1, release));
  CHECK(w.live_graphs() == 1 && w.retired() == 2 && g_live.count(b) && g_live.count(c));
  CHECK(!w.graph_destroyed(&g1, release));  // not twice
  // the last one destroyed releases them; the slots' current buffers stay
  CHECK(w.graph_destroyed(&g2, release));
  CHECK(w.live_graphs() == 0 && w.retired() == 0 && !g_live.count(b) && !g_live.count(c));
  CHECK(g_live.size() == 2 && g_live.count(d) && g_live.count(e));

  // a failed allocation leaves the slot empty (its old buffer released or retired)
  CHECK(w.grow(1, 100, 128, fail, release) == nullptr);
  CHECK(w.bytes(1) == 0 && w.buffer(1) == nullptr && !g_live.count(e));
  w.graph_created(&g3);
  CHECK(w.grow(0, 5000, 8192, fail, release) == nullptr && w.retired() == 1 && g_live.count(d));
  CHECK(w.graph_destroyed(&g3, release) && g_live.empty());

  // buffers freed during a capture: released at once when the capture made no graph, retired with
  // the graphs when it did (the graph may use them), and released with the last graph
  void *f = alloc(32), *h = alloc(32), *k = alloc(32);
  w.free_after_capture(f, release);  // no graph alive
  CHECK(!g_live.count(f) && w.retired() == 0);
  w.free_after_capture(nullptr, release);
  w.graph_created(&g1);               // the capture's graph
  w.free_after_capture(h, release);
  CHECK(g_live.count(h) && w.retired() == 1);
  w.graph_created(&g2);
  w.free_after_capture(k, release);
  CHECK(g_live.count(k) && w.retired() == 2);
  CHECK(w.graph_destroyed(&g1, release) && g_live.count(h) && g_live.count(k));
  CHECK(w.graph_destroyed(&g2, release) && !g_live.count(h) && !g_live.count(k));
  CHECK(g_live.empty() && w.retired() == 0);

  std::printf(g_fail ? "FAILED\n" : "ok\n");
  return g_fail;
}
