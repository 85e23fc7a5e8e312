// ws_ledger.hpp — the bookkeeping of the library's workspace slots and the graphs captured over
// them. Plain C++ (no HIP), so the rules can be checked on a machine without a GPU.
//
// A slot grows by allocating a larger buffer. A captured graph keeps the addresses its kernels
// were recorded with, so while any graph made by the library is alive an outgrown buffer is not
// freed but retired; the retired buffers are freed when the last such graph is destroyed. With no
// graph alive the old buffer is freed at once.
//
// Buffers the caller frees while a capture is open (arena_free_hip) are held back the same way:
// the capture's own kernels may have been recorded reading or writing them, so once the capture
// has produced a graph they are retired with the outgrown workspaces and freed with the last graph
// (a capture that produced no graph frees them at once).
#pragma once

#include <algorithm>
#include <cstddef>
#include <vector>

namespace plast {

template <int Slots>
class WorkspaceLedger {
 public:
  void *buffer(int slot) const { return buf_[slot]; }
  size_t bytes(int slot) const { return bytes_[slot]; }
  size_t live_graphs() const { return graphs_.size(); }
  size_t retired() const { return retired_.size(); }

  // The buffer of `slot` with room for `bytes`, after growing it to `want` bytes when it is
  // smaller: the old buffer is released (release(ptr)) or retired first, then alloc(want) returns
  // the new one (null on failure, which leaves the slot empty).
  template <class Alloc, class Release>
  void *grow(int slot, size_t bytes, size_t want, Alloc alloc, Release release) {
    if (bytes <= bytes_[slot]) return buf_[slot];
    if (buf_[slot]) {
      if (graphs_.empty())
        release(buf_[slot]);
      else
        retired_.push_back(buf_[slot]);
      buf_[slot] = nullptr;
      bytes_[slot] = 0;
    }
    void *fresh = alloc(want);
    if (!fresh) return nullptr;
    buf_[slot] = fresh;
    bytes_[slot] = want;
    return fresh;
  }

  void graph_created(const void *g) { graphs_.push_back(g); }

  // A buffer freed while a capture was open, handed over when the capture ends: retired when a
  // graph is alive (the capture's graph, just created, is), else released through release(ptr).
  template <class Release>
  void free_after_capture(void *p, Release release) {
    if (!p) return;
    if (graphs_.empty())
      release(p);
    else
      retired_.push_back(p);
  }

  // Forget graph `g` (false when the library did not make it); when it was the last one alive,
  // free the retired buffers through release(ptr).
  template <class Release>
  bool graph_destroyed(const void *g, Release release) {
    auto it = std::find(graphs_.begin(), graphs_.end(), g);
    if (it == graphs_.end()) return false;
    graphs_.erase(it);
    if (graphs_.empty()) {
      for (void *p : retired_) release(p);
      retired_.clear();
    }
    return true;
  }

 private:
  void *buf_[Slots] = {};
  size_t bytes_[Slots] = {};
  std::vector<const void *> graphs_;
  std::vector<void *> retired_;
};

}  // namespace plast
