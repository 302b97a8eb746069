// Host page pool of the paged KV cache (CPU only; never touches a device).
//
// Behaviour of src/moba_opt/cache_layout.py:23-148, restated as a flat C++
// state machine:
//   * table[b][w] is the physical page of logical page w of batch slot b
//     (-1 = unmapped), lengths[b] the tokens stored;
//   * free pages form a stack; the initial stack hands out page 0 first and
//     reset() pushes a slot's pages back in logical order, so the page freed
//     last is the next one handed out (cache_layout.py:37,92-98);
//   * appends are planned without touching the pool and committed by
//     version, so a failed plan (pool exhausted, past max_seq_len, bad ids)
//     changes nothing and a plan made before another commit is refused
//     (cache_layout.py:48-87);
//   * a decode step of a fixed set of slots adds one token to each; a slot
//     whose position starts a new page takes the next free page
//     (cache_layout.py:116-148).
// Planning is O(tokens appended) / O(slots stepped); no call copies the
// table.  Errors: MOBA_ERR_ARG (the caller's input; ValueError in Python) and
// MOBA_ERR_STALE (a plan older than the pool; RuntimeError in Python).
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/moba_hip.h"

void moba_set_error(const char* fmt, ...);

namespace {

struct PagePool {
  int batch = 0, max_len = 0, page = 0, num_pages = 0, chunk = 0, width = 0;
  std::vector<int32_t> table;    // [batch * width]
  std::vector<int32_t> lengths;  // [batch]
  std::vector<int32_t> free;     // [num_pages] stack storage; top = free[n_free - 1]
  int n_free = 0;
  int64_t version = 0;
};

PagePool* as_pool(void* p) { return static_cast<PagePool*>(p); }
const PagePool* as_pool(const void* p) { return static_cast<const PagePool*>(p); }

int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

int arg_error(const char* msg) {
  moba_set_error("%s", msg);
  return MOBA_ERR_ARG;
}

// Slot ids: each in [0, batch); nonempty; unique when `unique`.
// (cache_layout.py:41-52)
int check_ids(const PagePool& p, const int32_t* ids, int n, bool unique,
              std::vector<uint8_t>& seen) {
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= p.batch) return arg_error("sequence ID outside cache batch slots");
  if (n <= 0) return arg_error("nonempty unique sequence IDs required for append/reset");
  if (unique) {
    seen.assign(p.batch, 0);
    for (int i = 0; i < n; ++i) {
      if (seen[ids[i]]) return arg_error("nonempty unique sequence IDs required for append/reset");
      seen[ids[i]] = 1;
    }
  }
  return MOBA_OK;
}

}  // namespace

extern "C" int moba_pool_create(int batch, int max_seq_len, int page_size, int num_pages,
                                int chunk, void** out) {
  if (!out) return arg_error("pool_create: null output");
  *out = nullptr;
  if (batch <= 0 || max_seq_len <= 0 || page_size <= 0 || num_pages <= 0 || chunk <= 0)
    return arg_error("pool sizes must be positive integers");
  if (max_seq_len >= (1 << 30) || (int64_t)num_pages * page_size >= ((int64_t)1 << 31))
    return arg_error("cache exceeds int32 indexing capacity");
  PagePool* p = new (std::nothrow) PagePool;
  if (!p) return arg_error("pool_create: out of host memory");
  p->batch = batch; p->max_len = max_seq_len; p->page = page_size;
  p->num_pages = num_pages; p->chunk = chunk; p->width = ceil_div(max_seq_len, page_size);
  p->table.assign((size_t)batch * p->width, -1);
  p->lengths.assign(batch, 0);
  p->free.resize(num_pages);
  // stack bottom .. top = num_pages-1 .. 0: page 0 is handed out first
  for (int i = 0; i < num_pages; ++i) p->free[i] = num_pages - 1 - i;
  p->n_free = num_pages;
  *out = p;
  return MOBA_OK;
}

extern "C" void moba_pool_destroy(void* pool) { delete as_pool(pool); }

extern "C" int moba_pool_clone(const void* pool, void** out) {
  if (!pool || !out) return arg_error("pool_clone: null argument");
  PagePool* p = new (std::nothrow) PagePool(*as_pool(pool));
  if (!p) return arg_error("pool_clone: out of host memory");
  *out = p;
  return MOBA_OK;
}

extern "C" int moba_pool_assign(void* dst, const void* src) {
  PagePool* d = as_pool(dst);
  const PagePool* s = as_pool(src);
  if (!d || !s || d->batch != s->batch || d->width != s->width || d->num_pages != s->num_pages ||
      d->page != s->page || d->chunk != s->chunk || d->max_len != s->max_len)
    return arg_error("pool_assign: pools of different shapes");
  // element copies into the existing storage: views of table / lengths /
  // free stay valid
  std::memcpy(d->table.data(), s->table.data(), s->table.size() * sizeof(int32_t));
  std::memcpy(d->lengths.data(), s->lengths.data(), s->lengths.size() * sizeof(int32_t));
  std::memcpy(d->free.data(), s->free.data(), s->free.size() * sizeof(int32_t));
  d->n_free = s->n_free;
  d->version = s->version;
  return MOBA_OK;
}

extern "C" int moba_pool_info(const void* pool, int64_t* info) {
  const PagePool* p = as_pool(pool);
  if (!p || !info) return arg_error("pool_info: null argument");
  info[0] = p->batch; info[1] = p->max_len; info[2] = p->page; info[3] = p->num_pages;
  info[4] = p->chunk; info[5] = p->width; info[6] = p->version; info[7] = p->n_free;
  return MOBA_OK;
}

extern "C" const int32_t* moba_pool_table(const void* pool) {
  return pool ? as_pool(pool)->table.data() : nullptr;
}
extern "C" const int32_t* moba_pool_lengths(const void* pool) {
  return pool ? as_pool(pool)->lengths.data() : nullptr;
}
extern "C" const int32_t* moba_pool_free(const void* pool) {
  return pool ? as_pool(pool)->free.data() : nullptr;
}

extern "C" int moba_pool_set_free(void* pool, const int32_t* pages, int n) {
  PagePool* p = as_pool(pool);
  if (!p || (n && !pages)) return arg_error("pool_set_free: null argument");
  if (n != p->n_free) return arg_error("free page order must be a permutation of the free pages");
  std::vector<uint8_t> mark(p->num_pages, 0);
  for (int i = 0; i < p->n_free; ++i) mark[p->free[i]] = 1;
  for (int i = 0; i < n; ++i) {
    if (pages[i] < 0 || pages[i] >= p->num_pages || mark[pages[i]] != 1)
      return arg_error("free page order must be a permutation of the free pages");
    mark[pages[i]] = 2;
  }
  std::memcpy(p->free.data(), pages, (size_t)n * sizeof(int32_t));
  return MOBA_OK;
}

extern "C" int moba_pool_plan_append(const void* pool, const int32_t* ids, const int32_t* counts,
                                     int n, int32_t* token_seq, int32_t* token_pos,
                                     int32_t* closed, int closed_cap, int* n_closed,
                                     int32_t* grants, int grants_cap, int* n_grants,
                                     int32_t* new_lengths, int64_t* version) {
  const PagePool* p = as_pool(pool);
  if (!p || !n_closed || !n_grants || !version) return arg_error("pool_plan_append: null argument");
  std::vector<uint8_t> seen;
  if (int rc = check_ids(*p, ids, n, true, seen)) return rc;
  int64_t need = 0, n_cl = 0;
  for (int i = 0; i < n; ++i)
    if (counts[i] <= 0) return arg_error("append count must be a positive integer");
  for (int i = 0; i < n; ++i) {
    const int64_t old = p->lengths[ids[i]], now = old + counts[i];
    if (now > p->max_len) return arg_error("append exceeds max_seq_len");
    need += ceil_div(now, p->page) - ceil_div(old, p->page);
    n_cl += now / p->chunk - old / p->chunk;
  }
  if (need > p->n_free) return arg_error("KV page pool exhausted; cache was not modified");
  if (need > grants_cap || n_cl > closed_cap) return arg_error("pool_plan_append: output buffers too small");
  // pages are taken from the top of the stack in slot order, logical order
  int top = p->n_free, g = 0, c = 0;
  int64_t t = 0;
  for (int i = 0; i < n; ++i) {
    const int s = ids[i], old = p->lengths[s], now = old + counts[i];
    for (int w = ceil_div(old, p->page); w < ceil_div(now, p->page); ++w, ++g) {
      grants[3 * g] = s; grants[3 * g + 1] = w; grants[3 * g + 2] = p->free[--top];
    }
    if (token_seq && token_pos)
      for (int x = old; x < now; ++x, ++t) { token_seq[t] = s; token_pos[t] = x; }
    for (int ch = old / p->chunk; ch < now / p->chunk; ++ch, ++c) {
      closed[2 * c] = s; closed[2 * c + 1] = ch;
    }
    new_lengths[i] = now;
  }
  *n_grants = g;
  *n_closed = c;
  *version = p->version;
  return MOBA_OK;
}

extern "C" int moba_pool_commit_append(void* pool, const int32_t* ids, int n,
                                       const int32_t* new_lengths, const int32_t* grants,
                                       int n_grants, int64_t version) {
  PagePool* p = as_pool(pool);
  if (!p) return arg_error("pool_commit_append: null pool");
  if (version != p->version || n_grants > p->n_free) {
    moba_set_error("stale append plan");
    return MOBA_ERR_STALE;
  }
  // a plan of this version took the top n_grants pages in order
  for (int g = 0; g < n_grants; ++g)
    if (grants[3 * g + 2] != p->free[p->n_free - 1 - g]) {
      moba_set_error("stale append plan");
      return MOBA_ERR_STALE;
    }
  for (int g = 0; g < n_grants; ++g)
    p->table[(size_t)grants[3 * g] * p->width + grants[3 * g + 1]] = grants[3 * g + 2];
  p->n_free -= n_grants;
  for (int i = 0; i < n; ++i) p->lengths[ids[i]] = new_lengths[i];
  ++p->version;
  return MOBA_OK;
}

extern "C" int moba_pool_reset(void* pool, const int32_t* ids, int n) {
  PagePool* p = as_pool(pool);
  if (!p) return arg_error("pool_reset: null pool");
  std::vector<uint8_t> seen;
  if (int rc = check_ids(*p, ids, n, true, seen)) return rc;
  for (int i = 0; i < n; ++i) {
    int32_t* row = &p->table[(size_t)ids[i] * p->width];
    for (int w = 0; w < p->width; ++w)
      if (row[w] >= 0) { p->free[p->n_free++] = row[w]; row[w] = -1; }
    p->lengths[ids[i]] = 0;
  }
  ++p->version;
  return MOBA_OK;
}

extern "C" int moba_pool_check_ids(const void* pool, const int32_t* ids, int n, int unique) {
  const PagePool* p = as_pool(pool);
  if (!p) return arg_error("pool_check_ids: null pool");
  std::vector<uint8_t> seen;
  return check_ids(*p, ids, n, unique != 0, seen);
}

extern "C" int moba_pool_plan_step(const void* pool, const int32_t* ids, int n, int32_t* positions,
                                   int32_t* delta, int* n_grants, int64_t* version) {
  const PagePool* p = as_pool(pool);
  if (!p || !n_grants || !version || !delta || (n > 0 && !ids))
    return arg_error("pool_plan_step: null argument");
  // range only: a prepared step's ids were checked unique when it was made
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= p->batch) return arg_error("sequence ID outside cache batch slots");
  int need = 0;
  for (int i = 0; i < n; ++i) {
    const int pos = p->lengths[ids[i]];
    if (pos >= p->max_len) return arg_error("append exceeds max_seq_len");
    need += pos % p->page == 0;
  }
  if (need > p->n_free) return arg_error("KV page pool exhausted; cache was not modified");
  // delta [2][n]: logical page and physical page of row i, or -1 / -1
  int top = p->n_free;
  for (int i = 0; i < n; ++i) {
    const int pos = p->lengths[ids[i]];
    if (positions) positions[i] = pos;
    const bool fresh = pos % p->page == 0;
    delta[i] = fresh ? pos / p->page : -1;
    delta[n + i] = fresh ? p->free[--top] : -1;
  }
  *n_grants = need;
  *version = p->version;
  return MOBA_OK;
}

extern "C" int moba_pool_commit_step(void* pool, const int32_t* ids, int n, const int32_t* delta,
                                     int64_t version) {
  PagePool* p = as_pool(pool);
  if (!p || !delta || (n > 0 && !ids)) return arg_error("pool_commit_step: null argument");
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= p->batch) return arg_error("sequence ID outside cache batch slots");
  if (version != p->version) {
    moba_set_error("stale decode step plan");
    return MOBA_ERR_STALE;
  }
  int top = p->n_free;
  for (int i = 0; i < n; ++i)
    if (delta[n + i] >= 0 && (top <= 0 || delta[n + i] != p->free[--top])) {
      moba_set_error("stale decode step plan");
      return MOBA_ERR_STALE;
    }
  for (int i = 0; i < n; ++i) {
    if (delta[n + i] >= 0) {
      p->table[(size_t)ids[i] * p->width + delta[i]] = delta[n + i];
      --p->n_free;
    }
    ++p->lengths[ids[i]];
  }
  ++p->version;
  return MOBA_OK;
}
