// Host page pool for the paged K/V cache.
//
// The reference keeps one dense [left+right+1, D] shift buffer per slot and layer
// (parakeet/modules/cache.py:24-45) and a FIFO deque of free slots
// (parakeet/engine/scheduler.py:84,93-104).  Here every slot owns a ring of
// max_pages page ids; a page holds page_size consecutive frames of one stream for
// every layer.  Free pages sit in one FIFO queue: allocation pops the front, a
// freed page is pushed to the back, which is the deque discipline of the
// reference's slot pool applied to pages.
//
// One step of a slot (pk_pool_advance) covers frame positions [A, A+chunk):
//   1. evict: logical pages k whose last frame is older than the window that
//      ends at A+chunk, i.e. (k+1)*page_size <= A+chunk-window, go back to the
//      free queue (window = left + chunk, the dense cache length of cache.py:22);
//   2. allocate: logical pages up to (A+chunk-1)/page_size are taken from the
//      queue into ring entry k % max_pages;
//   3. the row {A, ring} is written out and A advances by chunk.
// A window of `window` frames touches at most max_pages = (window+P-2)/P + 1
// logical pages, so live pages never collide in the ring.

#include <cstdint>
#include <cstring>
#include <deque>
#include <mutex>
#include <new>
#include <vector>

#include "pk_common.h"

struct pk_pool {
  std::mutex mu;
  int32_t num_pages = 0;
  int32_t num_slots = 0;
  int32_t page_size = 0;
  int32_t left = 0;
  int32_t chunk = 0;
  int32_t window = 0;
  int32_t max_pages = 0;
  std::deque<int32_t> free_q;
  struct Slot {
    int64_t appended = 0;  // A: frames appended so far
    int64_t lo = 0;        // logical pages [lo, hi) are held
    int64_t hi = 0;
    uint64_t stamp = 0;    // last advance call that touched the slot
  };
  std::vector<Slot> slots;
  std::vector<int32_t> ring;  // [num_slots][max_pages]
  uint64_t call = 0;
};

namespace {

void free_slot_pages(pk_pool* p, int32_t s) {
  pk_pool::Slot& sl = p->slots[s];
  int32_t* ring = &p->ring[(size_t)s * p->max_pages];
  for (int64_t k = sl.lo; k < sl.hi; ++k) {
    int32_t& e = ring[k % p->max_pages];
    p->free_q.push_back(e);
    e = -1;
  }
  sl.lo = sl.hi = 0;
  sl.appended = 0;
}

}  // namespace

extern "C" {

int pk_pool_create(int32_t num_pages, int32_t num_slots, int32_t page_size, int32_t left,
                   int32_t chunk, const int32_t* page_order, pk_pool** out) {
  pk::clear_error();
  if (!out) return pk::fail(PK_ERR_INVALID, "pk_pool_create: out is NULL");
  *out = nullptr;
  if (page_size <= 0 || (page_size & (page_size - 1)) != 0)
    return pk::fail(PK_ERR_INVALID, "pk_pool_create: page_size %d is not a power of two",
                    page_size);
  if (left < 0 || chunk <= 0 || num_slots <= 0 || num_pages <= 0)
    return pk::fail(PK_ERR_INVALID,
                    "pk_pool_create: need left >= 0, chunk > 0, num_slots > 0, num_pages > 0 "
                    "(got %d, %d, %d, %d)",
                    left, chunk, num_slots, num_pages);
  const int32_t window = left + chunk;
  const int32_t max_pages = (window + page_size - 2) / page_size + 1;
  if ((int64_t)num_pages < (int64_t)num_slots * max_pages)
    return pk::fail(PK_ERR_INVALID,
                    "pk_pool_create: %d pages cannot hold %d slots of %d pages each",
                    num_pages, num_slots, max_pages);
  pk_pool* p = new (std::nothrow) pk_pool();
  if (!p) return pk::fail(PK_ERR_INVALID, "pk_pool_create: out of host memory");
  p->num_pages = num_pages;
  p->num_slots = num_slots;
  p->page_size = page_size;
  p->left = left;
  p->chunk = chunk;
  p->window = window;
  p->max_pages = max_pages;
  p->slots.assign(num_slots, pk_pool::Slot());
  p->ring.assign((size_t)num_slots * max_pages, -1);
  if (page_order) {
    std::vector<uint8_t> seen(num_pages, 0);
    for (int32_t i = 0; i < num_pages; ++i) {
      const int32_t pg = page_order[i];
      if (pg < 0 || pg >= num_pages || seen[pg]) {
        delete p;
        return pk::fail(PK_ERR_INVALID,
                        "pk_pool_create: page_order is not a permutation of 0..%d (entry %d = %d)",
                        num_pages - 1, i, pg);
      }
      seen[pg] = 1;
      p->free_q.push_back(pg);
    }
  } else {
    for (int32_t i = 0; i < num_pages; ++i) p->free_q.push_back(i);
  }
  *out = p;
  return PK_OK;
}

void pk_pool_destroy(pk_pool* pool) { delete pool; }

int pk_pool_max_pages(const pk_pool* pool) {
  if (!pool) return pk::fail(PK_ERR_INVALID, "pk_pool_max_pages: pool is NULL");
  return pool->max_pages;
}

int pk_pool_advance(pk_pool* pool, int32_t n, const int32_t* slots, int32_t* rows_out,
                    int32_t rows_stride) {
  pk::clear_error();
  if (!pool) return pk::fail(PK_ERR_INVALID, "pk_pool_advance: pool is NULL");
  if (n < 0 || (n > 0 && (!slots || !rows_out)))
    return pk::fail(PK_ERR_INVALID, "pk_pool_advance: bad batch (n=%d)", n);
  if (rows_stride < 1 + pool->max_pages)
    return pk::fail(PK_ERR_INVALID, "pk_pool_advance: rows_stride %d < 1 + max_pages %d",
                    rows_stride, pool->max_pages);
  std::lock_guard<std::mutex> lock(pool->mu);
  const uint64_t call = ++pool->call;
  // Validate the whole batch first so a bad call changes nothing.
  for (int32_t b = 0; b < n; ++b) {
    const int32_t s = slots[b];
    if (s < 0 || s >= pool->num_slots)
      return pk::fail(PK_ERR_INVALID, "pk_pool_advance: slot %d out of range [0, %d)", s,
                      pool->num_slots);
    if (pool->slots[s].stamp == call)
      return pk::fail(PK_ERR_STATE, "pk_pool_advance: slot %d appears twice in one step", s);
    pool->slots[s].stamp = call;
  }
  const int64_t P = pool->page_size;
  const int32_t M = pool->max_pages;
  for (int32_t b = 0; b < n; ++b) {
    const int32_t s = slots[b];
    pk_pool::Slot& sl = pool->slots[s];
    int32_t* ring = &pool->ring[(size_t)s * M];
    const int64_t end = sl.appended + pool->chunk;
    const int64_t start = end - pool->window;  // first position of the window
    while (sl.lo < sl.hi && (sl.lo + 1) * P <= start) {
      int32_t& e = ring[sl.lo % M];
      pool->free_q.push_back(e);
      e = -1;
      ++sl.lo;
    }
    if (sl.lo == sl.hi && sl.hi * P <= start) {
      // nothing held: the window starts at or after the next unallocated page
      sl.lo = sl.hi = start > 0 ? start / P : 0;
    }
    const int64_t need_hi = (end - 1) / P + 1;
    while (sl.hi < need_hi) {
      if (pool->free_q.empty())
        return pk::fail(PK_ERR_EXHAUSTED, "pk_pool_advance: page pool exhausted at slot %d", s);
      ring[sl.hi % M] = pool->free_q.front();
      pool->free_q.pop_front();
      ++sl.hi;
    }
    int32_t* row = rows_out + (size_t)b * rows_stride;
    row[0] = (int32_t)sl.appended;
    std::memcpy(row + 1, ring, sizeof(int32_t) * M);
    sl.appended = end;
  }
  return PK_OK;
}

int pk_pool_reset_slot(pk_pool* pool, int32_t slot) {
  pk::clear_error();
  if (!pool) return pk::fail(PK_ERR_INVALID, "pk_pool_reset_slot: pool is NULL");
  std::lock_guard<std::mutex> lock(pool->mu);
  if (slot < 0 || slot >= pool->num_slots)
    return pk::fail(PK_ERR_INVALID, "pk_pool_reset_slot: slot %d out of range [0, %d)", slot,
                    pool->num_slots);
  free_slot_pages(pool, slot);
  return PK_OK;
}

int pk_pool_reset_all(pk_pool* pool) {
  pk::clear_error();
  if (!pool) return pk::fail(PK_ERR_INVALID, "pk_pool_reset_all: pool is NULL");
  std::lock_guard<std::mutex> lock(pool->mu);
  for (int32_t s = 0; s < pool->num_slots; ++s) free_slot_pages(pool, s);
  return PK_OK;
}

int pk_pool_free_pages(const pk_pool* pool) {
  if (!pool) return pk::fail(PK_ERR_INVALID, "pk_pool_free_pages: pool is NULL");
  std::lock_guard<std::mutex> lock(const_cast<pk_pool*>(pool)->mu);
  return (int)pool->free_q.size();
}

int pk_pool_slot_info(const pk_pool* pool, int32_t slot, int64_t* appended, int32_t* ring_out) {
  pk::clear_error();
  if (!pool) return pk::fail(PK_ERR_INVALID, "pk_pool_slot_info: pool is NULL");
  std::lock_guard<std::mutex> lock(const_cast<pk_pool*>(pool)->mu);
  if (slot < 0 || slot >= pool->num_slots)
    return pk::fail(PK_ERR_INVALID, "pk_pool_slot_info: slot %d out of range [0, %d)", slot,
                    pool->num_slots);
  if (appended) *appended = pool->slots[slot].appended;
  if (ring_out)
    std::memcpy(ring_out, &pool->ring[(size_t)slot * pool->max_pages],
                sizeof(int32_t) * pool->max_pages);
  return PK_OK;
}

int pk_pool_free_list(const pk_pool* pool, int32_t* out, int32_t capacity) {
  pk::clear_error();
  if (!pool) return pk::fail(PK_ERR_INVALID, "pk_pool_free_list: pool is NULL");
  std::lock_guard<std::mutex> lock(const_cast<pk_pool*>(pool)->mu);
  const int32_t n = (int32_t)pool->free_q.size();
  if (out) {
    if (capacity < n)
      return pk::fail(PK_ERR_INVALID, "pk_pool_free_list: capacity %d < %d free pages", capacity,
                      n);
    int32_t i = 0;
    for (int32_t pg : pool->free_q) out[i++] = pg;
  }
  return n;
}

}  // extern "C"
