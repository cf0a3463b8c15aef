// velokv_radix.cpp -- prefix cache whose entries alias KV pages.
//
// RadixCache (radix_cache.rs:28-264) restated over the page handles of the host
// block manager (vk_bm_*): the same tree of token edges, the same edge splits,
// the same logical clock and coldest-first eviction, and the same results for
// insert and lookup. Bound to a block manager, the cache owns the handles it
// holds: a replaced or evicted handle is released there (its pages go back to
// the free list once no other handle references them), where the reference
// drops the handles that insert's eviction returns (radix_cache.rs:92, 250-262).
//
// vk_radix_cache_sequence is the engine's prefill / cache_sequence
// (engine.rs:435-494) with the pages of the longest cached prefix aliased
// (reference count + 1) instead of allocated again for every prompt.
#include "velokv.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <vector>

int vk_internal_set_error(int code, const char* msg);  // velokv_host.cpp

namespace {

int rfail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return vk_internal_set_error(code, buf);
}

struct RNode {
  std::vector<uint32_t> edge;            // tokens on the edge into this node
  std::map<uint32_t, int32_t> children;  // first token of the child's edge -> node
  bool has = false;                      // holds a handle
  uint64_t handle = 0;
  int64_t token_len = 0;
  uint64_t tick = 0;                     // last access (logical clock)
  uint64_t hits = 0;
};

size_t common_prefix(const uint32_t* a, size_t na, const std::vector<uint32_t>& b) {
  size_t n = 0;
  const size_t m = std::min(na, b.size());
  while (n < m && a[n] == b[n]) ++n;
  return n;
}

}  // namespace

struct vk_radix {
  std::vector<RNode> nodes;
  int64_t capacity = -1;  // < 0: no limit
  int64_t resident = 0;
  uint64_t clock = 1;
  vk_block_manager* bm = nullptr;

  vk_radix() { nodes.emplace_back(); }

  int32_t push(RNode&& n) {
    nodes.push_back(std::move(n));
    return (int32_t)nodes.size() - 1;
  }

  // split the edge of child (reached from parent) after `at` tokens; the new
  // node takes the first part (split_child, radix_cache.rs:223-242)
  int32_t split(int32_t parent, int32_t child, size_t at) {
    const uint32_t old_first = nodes[(size_t)child].edge[0];
    std::vector<uint32_t> prefix(nodes[(size_t)child].edge.begin(), nodes[(size_t)child].edge.begin() + (long)at);
    nodes[(size_t)child].edge.erase(nodes[(size_t)child].edge.begin(), nodes[(size_t)child].edge.begin() + (long)at);
    const uint32_t new_first = nodes[(size_t)child].edge[0];
    RNode s;
    s.edge = std::move(prefix);
    s.children[new_first] = child;
    s.tick = clock;
    s.hits = nodes[(size_t)child].hits;
    const int32_t sid = push(std::move(s));
    nodes[(size_t)parent].children[old_first] = sid;
    return sid;
  }

  // node for exactly `tokens`, created or split as needed (insert_from)
  int32_t insert_path(const uint32_t* tokens, size_t n) {
    int32_t node = 0;
    while (n > 0) {
      auto it = nodes[(size_t)node].children.find(tokens[0]);
      if (it == nodes[(size_t)node].children.end()) {
        RNode c;
        c.edge.assign(tokens, tokens + n);
        c.tick = clock;
        const int32_t cid = push(std::move(c));
        nodes[(size_t)node].children[tokens[0]] = cid;
        return cid;
      }
      const int32_t child = it->second;
      const size_t common = common_prefix(tokens, n, nodes[(size_t)child].edge);
      if (common == nodes[(size_t)child].edge.size()) {
        node = child;
        tokens += common;
        n -= common;
        continue;
      }
      const int32_t sid = split(node, child, common);
      if (common == n) return sid;
      node = sid;
      tokens += common;
      n -= common;
    }
    return node;
  }

  int release(uint64_t handle) {
    return bm ? vk_bm_release(bm, handle) : VK_OK;
  }

  // coldest first (stable by node index on equal ticks), until `tokens` are freed
  int evict(int64_t tokens, std::vector<uint64_t>* out) {
    std::vector<std::pair<uint64_t, int32_t>> order;
    for (size_t i = 0; i < nodes.size(); ++i)
      if (nodes[i].has) order.emplace_back(nodes[i].tick, (int32_t)i);
    std::stable_sort(order.begin(), order.end(),
                     [](const std::pair<uint64_t, int32_t>& a, const std::pair<uint64_t, int32_t>& b) {
                       return a.first < b.first;
                     });
    int64_t freed = 0;
    for (const auto& e : order) {
      if (freed >= tokens) break;
      RNode& nd = nodes[(size_t)e.second];
      nd.has = false;
      resident -= nd.token_len;
      freed += nd.token_len;
      if (out) out->push_back(nd.handle);
      int rc = release(nd.handle);
      if (rc) return rc;
    }
    return VK_OK;
  }

  int evict_to_capacity() {
    if (capacity < 0 || resident <= capacity) return VK_OK;
    return evict(resident - capacity, nullptr);
  }
};

extern "C" int vk_radix_create(vk_block_manager* bm, int64_t capacity_tokens, vk_radix** out) {
  if (!out) return rfail(VK_ERR_BAD_ARG, "out is null");
  auto* rc = new vk_radix();
  rc->bm = bm;
  rc->capacity = capacity_tokens < 0 ? -1 : capacity_tokens;
  *out = rc;
  return VK_OK;
}

extern "C" int vk_radix_destroy(vk_radix* rc) {
  if (!rc) return VK_OK;
  int status = VK_OK;
  for (RNode& n : rc->nodes)
    if (n.has) {
      const int r = rc->release(n.handle);
      if (r && status == VK_OK) status = r;
    }
  delete rc;
  return status;
}

extern "C" int vk_radix_insert(vk_radix* rc, const uint32_t* tokens, int32_t n_tokens, uint64_t handle,
                               uint64_t* replaced, int32_t* has_replaced) {
  if (!rc) return rfail(VK_ERR_BAD_ARG, "null cache");
  if (n_tokens < 0 || (n_tokens > 0 && !tokens)) return rfail(VK_ERR_BAD_ARG, "bad token array");
  if (rc->bm) {
    int32_t n_pages = 0;
    int r = vk_bm_pages(rc->bm, handle, nullptr, 0, &n_pages);
    if (r) return r;
  }
  rc->clock += 1;
  RNode& root = rc->nodes[0];
  root.tick = rc->clock;
  root.hits += 1;
  const int32_t leaf = rc->insert_path(tokens, (size_t)n_tokens);
  RNode& lf = rc->nodes[(size_t)leaf];
  const bool had = lf.has;
  const uint64_t old = lf.handle;
  const int64_t old_len = lf.token_len;
  lf.has = true;
  lf.handle = handle;
  lf.token_len = n_tokens;
  lf.tick = rc->clock;
  lf.hits += 1;
  if (had) rc->resident -= old_len;
  rc->resident += n_tokens;
  if (has_replaced) *has_replaced = had ? 1 : 0;
  if (replaced) *replaced = had ? old : 0;
  if (had && old != handle) {
    int r = rc->release(old);
    if (r) return r;
  }
  return rc->evict_to_capacity();
}

extern "C" int vk_radix_lookup(vk_radix* rc, const uint32_t* tokens, int32_t n_tokens, int32_t* matched,
                               uint64_t* handle, int32_t* has_handle) {
  if (!rc || !matched || !handle || !has_handle) return rfail(VK_ERR_BAD_ARG, "null argument");
  if (n_tokens < 0 || (n_tokens > 0 && !tokens)) return rfail(VK_ERR_BAD_ARG, "bad token array");
  rc->clock += 1;
  const uint64_t tick = rc->clock;
  int32_t node = 0;
  size_t cursor = 0;
  bool best = rc->nodes[0].has;
  size_t best_len = 0;
  uint64_t best_handle = rc->nodes[0].handle;
  rc->nodes[0].tick = tick;
  rc->nodes[0].hits += 1;
  while (cursor < (size_t)n_tokens) {
    auto it = rc->nodes[(size_t)node].children.find(tokens[cursor]);
    if (it == rc->nodes[(size_t)node].children.end()) break;
    const int32_t child = it->second;
    const RNode& c = rc->nodes[(size_t)child];
    const size_t m = common_prefix(tokens + cursor, (size_t)n_tokens - cursor, c.edge);
    if (m < c.edge.size()) break;
    cursor += m;
    node = child;
    rc->nodes[(size_t)node].tick = tick;
    rc->nodes[(size_t)node].hits += 1;
    if (rc->nodes[(size_t)node].has) {
      best = true;
      best_len = cursor;
      best_handle = rc->nodes[(size_t)node].handle;
    }
  }
  *matched = best ? (int32_t)best_len : 0;
  *has_handle = best ? 1 : 0;
  *handle = best ? best_handle : 0;
  return VK_OK;
}

extern "C" int vk_radix_len(const vk_radix* rc, int32_t* out) {
  if (!rc || !out) return rfail(VK_ERR_BAD_ARG, "null argument");
  int32_t n = 0;
  for (const RNode& nd : rc->nodes) n += nd.has ? 1 : 0;
  *out = n;
  return VK_OK;
}

extern "C" int vk_radix_resident_tokens(const vk_radix* rc, int64_t* out) {
  if (!rc || !out) return rfail(VK_ERR_BAD_ARG, "null argument");
  *out = rc->resident;
  return VK_OK;
}

extern "C" int vk_radix_capacity_tokens(const vk_radix* rc, int64_t* out) {
  if (!rc || !out) return rfail(VK_ERR_BAD_ARG, "null argument");
  *out = rc->capacity;
  return VK_OK;
}

extern "C" int vk_radix_set_capacity(vk_radix* rc, int64_t capacity_tokens) {
  if (!rc) return rfail(VK_ERR_BAD_ARG, "null cache");
  rc->capacity = capacity_tokens < 0 ? -1 : capacity_tokens;
  return rc->evict_to_capacity();
}

extern "C" int vk_radix_evict_coldest(vk_radix* rc, int64_t tokens, uint64_t* evicted, int32_t cap, int32_t* n_out) {
  if (!rc) return rfail(VK_ERR_BAD_ARG, "null cache");
  std::vector<uint64_t> ev;
  int r = rc->evict(tokens, &ev);
  if (n_out) *n_out = (int32_t)ev.size();
  if (evicted) {
    if ((int64_t)ev.size() > cap) return rfail(VK_ERR_BAD_ARG, "output capacity %d < %zu handles", cap, ev.size());
    std::copy(ev.begin(), ev.end(), evicted);
  }
  return r;
}

extern "C" int vk_radix_cache_sequence(vk_radix* rc, const uint32_t* tokens, int32_t n_tokens, uint64_t seq_handle,
                                       uint64_t cache_handle, int32_t* matched_tokens, uint32_t* pages_out,
                                       int32_t cap, int32_t* n_pages, int32_t* cow_src, int32_t* cow_dst,
                                       int32_t* has_cow) {
  if (!rc || !matched_tokens || !cow_src || !cow_dst || !has_cow) return rfail(VK_ERR_BAD_ARG, "null argument");
  if (!rc->bm) return rfail(VK_ERR_UNSUPPORTED, "cache_sequence needs a cache bound to a block manager");
  if (seq_handle == cache_handle) return rfail(VK_ERR_BAD_ARG, "seq_handle and cache_handle must differ");
  int32_t m = 0, has = 0;
  uint64_t h = 0;
  int r = vk_radix_lookup(rc, tokens, n_tokens, &m, &h, &has);
  if (r) return r;
  *matched_tokens = m;
  *has_cow = 0;
  *cow_src = *cow_dst = -1;
  // the sequence's pages: the cached prefix's pages aliased, fresh ones after it
  if (has && m > 0) r = vk_bm_fork(rc->bm, h, seq_handle, m, n_tokens, nullptr, 0, nullptr);
  else r = vk_bm_allocate(rc->bm, seq_handle, n_tokens, nullptr, 0, nullptr);
  if (r) return r;
  if (m < n_tokens) {
    // the prompt continues inside the prefix's partially filled last page: give
    // the sequence its own copy of that page before it is written
    int32_t block_size = 0;
    r = vk_bm_block_size(rc->bm, &block_size);
    if (r) return r;
    if (has && m % block_size) {
      int32_t copied = 0;
      r = vk_bm_cow(rc->bm, seq_handle, m / block_size, cow_src, cow_dst, &copied);
      if (r) return r;
      *has_cow = copied;
    }
    // cache the whole prompt under its own handle (all of the sequence's pages)
    r = vk_bm_fork(rc->bm, seq_handle, cache_handle, n_tokens, n_tokens, nullptr, 0, nullptr);
    if (r) return r;
    r = vk_radix_insert(rc, tokens, n_tokens, cache_handle, nullptr, nullptr);
    if (r) return r;
  }
  return vk_bm_pages(rc->bm, seq_handle, pages_out, cap, n_pages);
}
