// kv_pool.cc - the host page-table controller (granite4_kv_pool.h): paged KV
// pool bookkeeping and session slots, producing the position -> arena-row
// tables the append / attention kernels index through.
//
// Allocation invariant (as the reference's, kv_pool.cc:5-10): a page is
// allocated iff it has a reference or is cached. A cached page at ref count 0
// is "retained": still shareable by a later prompt with the same prefix, and
// evictable (least recently used first) when the free list runs dry.
//
// Data structures (this build's choices): the retained pages sit in an
// ordered set keyed by their last-use tick, so eviction is O(log n) instead of
// a scan over the pool; the shared count is kept incrementally; each
// sequence caches its chained prefix keys, so keying page i costs one page
// hash instead of rehashing pages 0..i-1. Observable results are the
// reference's: the same page ids (a LIFO free list over [0, num_pages),
// highest id first), the same eviction order, the same counts.

#include "granite4_kv_pool.h"

#include <algorithm>
#include <climits>
#include <cstdint>
#include <new>

namespace granite4 {

namespace {

// Page keys: 64-bit FNV-1a over the page's token ids (one step per 32-bit
// id), seeded with the key of the pages before it. Any hash would do (the
// cache verifies tokens on lookup); this one is the reference's
// (kv_pool.cc:19-22, 69-77), so keys agree across the two implementations.
constexpr std::uint64_t kKeySeed = 1469598103934665603ULL;
constexpr std::uint64_t kKeyPrime = 1099511628211ULL;

std::uint64_t key_step(const std::uint32_t* ids, std::size_t n, std::uint64_t h) {
  for (std::size_t i = 0; i < n; ++i) {
    h ^= static_cast<std::uint64_t>(ids[i]);
    h *= kKeyPrime;
  }
  return h;
}

constexpr std::size_t kNoIndex = static_cast<std::size_t>(-1);

}  // namespace

// ---------------------------------------------------------------------------
// Layout and sizing (kv_pool.cc:28-64).
// ---------------------------------------------------------------------------

KvLayout KvLayout::make(std::size_t layers, std::size_t kv_heads, std::size_t head_dim) {
  KvLayout l;
  l.num_layers = layers;
  l.num_kv_heads = kv_heads;
  l.head_dim = head_dim;
  l.bytes_per_token = 2 * layers * kv_heads * head_dim;
  return l;
}

std::size_t KvLayout::offset(std::size_t tokens_per_page, std::size_t token_local,
                             std::size_t layer, int kv, std::size_t head, std::size_t dim) const {
  if (token_local >= tokens_per_page || layer >= num_layers || (kv != 0 && kv != 1) ||
      head >= num_kv_heads || dim >= head_dim)
    return kNoIndex;
  const std::size_t per_kv = num_kv_heads * head_dim;
  return token_local * bytes_per_token + (2 * layer + static_cast<std::size_t>(kv)) * per_kv +
         head * head_dim + dim;
}

KvPoolConfig KvPoolConfig::from_budget(const KvLayout& layout, std::size_t tokens_per_page,
                                       std::size_t budget_bytes) {
  KvPoolConfig c;
  c.layout = layout;
  c.tokens_per_page = tokens_per_page;
  c.budget_bytes = budget_bytes;
  c.page_bytes = tokens_per_page * layout.bytes_per_token;
  c.num_pages = c.page_bytes > 0 ? budget_bytes / c.page_bytes : 0;
  return c;
}

// ---------------------------------------------------------------------------
// PagedKV.
// ---------------------------------------------------------------------------

PagedKV::PagedKV(KvPoolConfig config) : config_(config), pages_(config.num_pages) {
  free_.reserve(config_.num_pages);
  for (std::size_t i = 0; i < config_.num_pages; ++i) free_.push_back(i);
}

bool PagedKV::valid(int seq) const {
  return seq >= 0 && seq < static_cast<int>(seqs_.size()) && seqs_[seq].live;
}

void PagedKV::take_ref(std::size_t page) {
  Page& p = pages_[page];
  if (p.refs == 0 && p.cached) lru_.erase({p.tick, page});  // retained -> in use
  ++p.refs;
  if (p.refs == 2) ++shared_;
}

void PagedKV::free_page(std::size_t page) {
  Page& p = pages_[page];
  p.tokens.clear();
  p.key = 0;
  p.tick = 0;
  p.cached = false;
  free_.push_back(page);
}

void PagedKV::put_ref(std::size_t page) {
  Page& p = pages_[page];
  if (p.refs == 0) return;
  if (p.refs == 2) --shared_;
  if (--p.refs > 0) return;
  if (p.cached) {
    lru_.insert({p.tick, page});  // retained for a later prompt
  } else {
    free_page(page);
  }
}

// Removes a page from the cache; an unreferenced page goes back to the free
// list (the reference leaves such a page allocated and unreachable).
void PagedKV::uncache(std::size_t page) {
  Page& p = pages_[page];
  if (!p.cached) return;
  if (p.refs == 0) lru_.erase({p.tick, page});
  p.cached = false;
  if (p.refs == 0) free_page(page);
}

std::size_t PagedKV::evict_lru() {
  if (lru_.empty()) return pages_.size();
  const std::size_t page = lru_.begin()->second;
  lru_.erase(lru_.begin());
  Page& p = pages_[page];
  const auto it = cache_.find(p.key);
  if (it != cache_.end() && it->second == page) cache_.erase(it);
  free_page(page);
  ++evicted_;
  return page;
}

// Key of the first page_index pages of s (pages before the tail are full).
std::uint64_t PagedKV::prefix_key(Seq& s, std::size_t page_index) {
  if (s.chain.empty()) s.chain.push_back(kKeySeed);
  while (s.chain.size() <= page_index) {
    const std::size_t j = s.chain.size() - 1;
    const Page& p = pages_[s.pages[j]];
    s.chain.push_back(key_step(p.tokens.data(), p.tokens.size(), s.chain[j]));
  }
  return s.chain[page_index];
}

int PagedKV::create_sequence() {
  if (live_ >= std::max<std::size_t>(1, config_.num_pages)) return -1;
  Seq s;
  s.live = true;
  seqs_.push_back(std::move(s));
  ++live_;
  return static_cast<int>(seqs_.size()) - 1;
}

std::size_t PagedKV::match_prefix(int seq, const Tokens& tokens) {
  if (!valid(seq) || seqs_[seq].filled != 0) return 0;  // only an empty sequence adopts
  Seq& s = seqs_[seq];
  const std::size_t B = config_.tokens_per_page;
  std::size_t pos = 0;
  while (pos + B <= tokens.size()) {
    const std::size_t i = pos / B;
    const std::uint64_t key = key_step(tokens.data() + pos, B, prefix_key(s, i));
    const auto it = cache_.find(key);
    if (it == cache_.end()) break;
    const std::size_t page = it->second;
    const Page& c = pages_[page];
    if (c.tokens.size() != B || !std::equal(c.tokens.begin(), c.tokens.end(), tokens.begin() + pos))
      break;  // a colliding key: stop at the longest verified prefix
    take_ref(page);
    s.pages.push_back(page);
    pages_[page].tick = ++tick_;
    s.chain.resize(i + 1);
    s.chain.push_back(key);
    s.filled += B;
    pos += B;
  }
  return pos;
}

bool PagedKV::reserve(int seq, std::size_t token_count, const Tokens& tokens) {
  if (!valid(seq) || tokens.size() < token_count) return false;
  Seq& s = seqs_[seq];
  if (token_count <= s.filled) return true;
  const std::size_t B = config_.tokens_per_page;
  const std::size_t held = s.pages.size() * B;  // logical window of the pages held
  const std::size_t beyond = token_count > held ? token_count - held : 0;
  const std::size_t need = (beyond + B - 1) / B;
  // Fail before changing anything (no partial eviction).
  if (free_.size() + lru_.size() < need) return false;
  if (s.filled < held && pages_[s.pages.back()].cached) {
    // The sequence was truncated inside a cached (shared, full) page: its
    // rows already hold the page's tokens, so growing back over them is
    // bookkeeping only. Different tokens would overwrite shared rows: refused.
    const Page& p = pages_[s.pages.back()];
    const std::size_t base = held - B, upto = std::min(held, token_count);
    for (std::size_t i = s.filled; i < upto; ++i)
      if (p.tokens[i - base] != tokens[i]) return false;
  }
  while (free_.size() < need) evict_lru();

  if (s.filled < held) {  // top up the partial tail page first: pages stay dense
    Page& p = pages_[s.pages.back()];
    const std::size_t upto = std::min(held, token_count);
    if (!p.cached)  // a cached tail already holds these ids (checked above)
      p.tokens.insert(p.tokens.end(), tokens.begin() + s.filled, tokens.begin() + upto);
    s.filled = upto;
  }
  while (s.filled < token_count) {
    const std::size_t page = free_.back();
    free_.pop_back();
    Page& p = pages_[page];
    const std::size_t hi = std::min(s.filled + B, token_count);
    p.tokens.assign(tokens.begin() + s.filled, tokens.begin() + hi);
    p.key = 0;
    p.tick = 0;
    p.cached = false;
    p.refs = 0;
    take_ref(page);
    s.pages.push_back(page);
    s.filled = hi;
  }
  return true;
}

bool PagedKV::mark_written(int seq, std::size_t page_index) {
  if (!valid(seq)) return false;
  Seq& s = seqs_[seq];
  if (page_index >= s.pages.size()) return false;
  const std::size_t page = s.pages[page_index];
  Page& p = pages_[page];
  if (p.refs != 1 || p.tokens.size() != config_.tokens_per_page) return false;
  const std::uint64_t key = key_step(p.tokens.data(), p.tokens.size(), prefix_key(s, page_index));
  const auto it = cache_.find(key);
  if (it != cache_.end() && it->second != page) uncache(it->second);  // displaced by a collision
  cache_[key] = page;
  p.key = key;
  p.cached = true;
  p.tick = ++tick_;
  return true;
}

std::array<std::size_t, 2> PagedKV::locate(int seq, std::size_t token) const {
  if (!valid(seq) || token >= seqs_[seq].filled) return {kNoIndex, kNoIndex};
  const std::size_t B = config_.tokens_per_page;
  return {seqs_[seq].pages[token / B], token % B};
}

bool PagedKV::row_table(int seq, std::size_t n, int* out) const {
  if (!valid(seq) || out == nullptr || n > seqs_[seq].filled) return false;
  const Seq& s = seqs_[seq];
  const std::size_t B = config_.tokens_per_page;
  for (std::size_t i = 0; i < n; ++i) out[i] = static_cast<int>(s.pages[i / B] * B + i % B);
  return true;
}

void PagedKV::reset_sequence(int seq) {
  if (!valid(seq)) return;
  Seq& s = seqs_[seq];
  for (const std::size_t page : s.pages) put_ref(page);
  s.pages.clear();
  s.chain.clear();
  s.filled = 0;
}

void PagedKV::truncate_sequence(int seq, std::size_t n_tokens) {
  if (!valid(seq)) return;
  Seq& s = seqs_[seq];
  const std::size_t B = config_.tokens_per_page;
  const std::size_t keep = (n_tokens + B - 1) / B;
  const bool dropped = s.pages.size() > keep;
  for (std::size_t i = keep; i < s.pages.size(); ++i) put_ref(s.pages[i]);
  if (dropped) s.pages.resize(keep);
  s.filled = std::min(s.filled, n_tokens);
  if (keep > 0 && !s.pages.empty()) {
    Page& last = pages_[s.pages.back()];
    if (last.cached) {
      // A cached page is full and shared: its ids stay whole. When pages were
      // dropped the sequence keeps the whole page (as the reference does);
      // otherwise the count is trimmed, and reserve regrows it only with the
      // page's own tokens.
      if (dropped) s.filled = s.pages.size() * B;
    } else {
      const std::size_t in_last = s.filled > (s.pages.size() - 1) * B ? s.filled - (s.pages.size() - 1) * B : 0;
      if (last.tokens.size() > in_last) last.tokens.resize(in_last);
    }
  }
  const std::size_t full = s.filled / B;  // chained keys stay valid for full pages only
  if (s.chain.size() > full + 1) s.chain.resize(full + 1);
}

void PagedKV::release(int seq) {
  if (!valid(seq)) return;
  reset_sequence(seq);
  seqs_[seq].live = false;
  --live_;
}

void PagedKV::clear() {
  seqs_.clear();
  cache_.clear();
  lru_.clear();
  for (Page& p : pages_) p = Page{};
  free_.clear();
  for (std::size_t i = 0; i < config_.num_pages; ++i) free_.push_back(i);
  tick_ = 0;
  evicted_ = 0;
  shared_ = 0;
  live_ = 0;
}

const std::vector<std::size_t>& PagedKV::block_table(int seq) const {
  static const std::vector<std::size_t> kEmpty;
  return valid(seq) ? seqs_[seq].pages : kEmpty;
}

std::size_t PagedKV::sequence_tokens(int seq) const { return valid(seq) ? seqs_[seq].filled : 0; }

std::size_t PagedKV::ref_count(std::size_t page_id) const {
  return page_id < pages_.size() ? static_cast<std::size_t>(pages_[page_id].refs) : 0;
}

bool PagedKV::page_in_cache(std::size_t page_id) const {
  return page_id < pages_.size() && pages_[page_id].cached;
}

// ---------------------------------------------------------------------------
// KvPoolController (kv_pool_controller.cc).
// ---------------------------------------------------------------------------

KvPoolController::KvPoolController(KvPoolConfig config) : pool_(config) {}
KvPoolController::~KvPoolController() { shutdown(); }

const KvPoolController::Slot* KvPoolController::slot_of(int slot) const {
  if (slot < 0 || slot >= static_cast<int>(slots_.size())) return nullptr;
  return &slots_[slot];
}

int KvPoolController::new_slot() {
  // An idle slot keeps its live pool sequence (emptied, not released), so
  // slot ids stay stable across requests.
  for (std::size_t i = 0; i < slots_.size(); ++i) {
    if (!slots_[i].in_use) {
      slots_[i].marked = 0;
      slots_[i].reused = 0;
      slots_[i].in_use = true;
      return static_cast<int>(i);
    }
  }
  const int seq = pool_.create_sequence();
  if (seq < 0) return -1;
  slots_.push_back(Slot{seq, 0, 0, true});
  return static_cast<int>(slots_.size()) - 1;
}

void KvPoolController::release_slot(int slot) {
  if (slot_of(slot) == nullptr) return;
  Slot& s = slots_[slot];
  pool_.reset_sequence(s.seq);  // private pages freed, cached ones retained
  s.in_use = false;
  s.marked = 0;
  s.reused = 0;
}

void KvPoolController::shutdown() {
  pool_.clear();
  slots_.clear();
}

void KvPoolController::mark_full(Slot& s, std::size_t n_tokens) {
  const std::size_t full = n_tokens / pool_.page_rows();
  for (std::size_t i = s.marked; i < full; ++i) pool_.mark_written(s.seq, i);
  s.marked = std::max(s.marked, full);
}

KvPoolController::Prefill KvPoolController::prefill(int slot, const PagedKV::Tokens& prompt) {
  Prefill r;
  if (slot_of(slot) == nullptr) return r;
  Slot& s = slots_[slot];
  pool_.reset_sequence(s.seq);
  s.marked = 0;
  s.reused = pool_.match_prefix(s.seq, prompt);
  if (!pool_.reserve(s.seq, prompt.size(), prompt)) {
    pool_.reset_sequence(s.seq);  // give back the adopted pages too
    s.in_use = false;
    s.reused = 0;
    return r;
  }
  s.in_use = true;
  mark_full(s, prompt.size());
  r.seq = s.seq;
  r.reused = s.reused;
  r.ok = true;
  return r;
}

void KvPoolController::commit(int slot, const PagedKV::Tokens& all_tokens) {
  const Slot* c = slot_of(slot);
  if (c == nullptr || !c->in_use) return;
  Slot& s = slots_[slot];
  if (all_tokens.size() <= pool_.sequence_tokens(s.seq)) return;
  if (!pool_.reserve(s.seq, all_tokens.size(), all_tokens)) return;
  mark_full(s, all_tokens.size());
}

int KvPoolController::open_slot() { return new_slot(); }

bool KvPoolController::ensure(int slot, std::size_t n_tokens) {
  const Slot* s = slot_of(slot);
  if (s == nullptr || !s->in_use) return false;
  if (n_tokens <= pool_.sequence_tokens(s->seq)) return true;
  // Resident pages never enter the cache, so their token ids are placeholders.
  const PagedKV::Tokens ids(n_tokens, 0u);
  return pool_.reserve(s->seq, n_tokens, ids);
}

void KvPoolController::trim(int slot, std::size_t n_tokens) {
  const Slot* s = slot_of(slot);
  if (s != nullptr && s->in_use) pool_.truncate_sequence(s->seq, n_tokens);
}

void KvPoolController::drop(int slot) {
  const Slot* c = slot_of(slot);
  if (c == nullptr || !c->in_use) return;
  Slot& s = slots_[slot];
  pool_.reset_sequence(s.seq);
  s.marked = 0;
  s.reused = 0;
}

std::size_t KvPoolController::slot_pages(int slot) const {
  const Slot* s = slot_of(slot);
  return (s != nullptr && s->in_use) ? pool_.block_table(s->seq).size() : 0;
}

std::size_t KvPoolController::pages_missing(int slot, std::size_t n_tokens) const {
  const std::size_t B = pool_.page_rows();
  const std::size_t want = (n_tokens + B - 1) / B;
  const std::size_t have = slot_pages(slot);
  return want > have ? want - have : 0;
}

bool KvPoolController::row_table(int slot, std::size_t n, int* out) const {
  const Slot* s = slot_of(slot);
  return s != nullptr && s->in_use && pool_.row_table(s->seq, n, out);
}

std::size_t KvPoolController::committed(int slot) const {
  const Slot* s = slot_of(slot);
  return (s != nullptr && s->in_use) ? pool_.sequence_tokens(s->seq) : 0;
}

std::size_t KvPoolController::last_reused(int slot) const {
  const Slot* s = slot_of(slot);
  return s != nullptr ? s->reused : 0;
}

}  // namespace granite4

// ---------------------------------------------------------------------------
// C ABI.
// ---------------------------------------------------------------------------

using granite4::KvLayout;
using granite4::KvPoolConfig;
using granite4::KvPoolController;
using granite4::PagedKV;

namespace {

KvPoolConfig config_of(size_t layers, size_t kv_heads, size_t head_dim, size_t tpp, size_t budget) {
  return KvPoolConfig::from_budget(KvLayout::make(layers, kv_heads, head_dim), tpp, budget);
}

PagedKV::Tokens ids_of(const uint32_t* p, size_t n) {
  return p != nullptr ? PagedKV::Tokens(p, p + n) : PagedKV::Tokens();
}

size_t stat_of(const PagedKV& p, int which) {
  switch (which) {
    case GRANITE4_KV_POOL_PAGES: return p.pool_pages();
    case GRANITE4_KV_FREE_PAGES: return p.free_pages();
    case GRANITE4_KV_USED_PAGES: return p.used_pages();
    case GRANITE4_KV_SHARED_PAGES: return p.shared_pages();
    case GRANITE4_KV_CACHED_PAGES: return p.cached_pages();
    case GRANITE4_KV_RETAINED_PAGES: return p.retained_pages();
    case GRANITE4_KV_EVICTED_PAGES: return p.evicted_pages();
    case GRANITE4_KV_LIVE_SEQUENCES: return p.live_sequences();
    case GRANITE4_KV_CAPACITY_TOKENS: return p.capacity_tokens();
    case GRANITE4_KV_PAGE_BYTES: return p.config().page_bytes;
    case GRANITE4_KV_TOKENS_PER_PAGE: return p.page_rows();
    default: return SIZE_MAX;
  }
}

}  // namespace

extern "C" {

size_t granite4_kv_layout_offset(size_t layers, size_t kv_heads, size_t head_dim,
                                 size_t tokens_per_page, size_t token_local, size_t layer, int kv,
                                 size_t head, size_t dim) {
  return KvLayout::make(layers, kv_heads, head_dim)
      .offset(tokens_per_page, token_local, layer, kv, head, dim);
}

void* granite4_kv_pool_create(size_t layers, size_t kv_heads, size_t head_dim,
                              size_t tokens_per_page, size_t budget_bytes) {
  if (tokens_per_page == 0) return nullptr;
  return new (std::nothrow) PagedKV(config_of(layers, kv_heads, head_dim, tokens_per_page, budget_bytes));
}
void granite4_kv_pool_destroy(void* pool) { delete static_cast<PagedKV*>(pool); }
size_t granite4_kv_pool_stat(const void* pool, int which) {
  return stat_of(*static_cast<const PagedKV*>(pool), which);
}
int granite4_kv_pool_create_sequence(void* pool) {
  return static_cast<PagedKV*>(pool)->create_sequence();
}
size_t granite4_kv_pool_match_prefix(void* pool, int seq, const uint32_t* tokens, size_t n) {
  return static_cast<PagedKV*>(pool)->match_prefix(seq, ids_of(tokens, n));
}
int granite4_kv_pool_reserve(void* pool, int seq, size_t token_count, const uint32_t* tokens,
                             size_t n) {
  return static_cast<PagedKV*>(pool)->reserve(seq, token_count, ids_of(tokens, n)) ? 1 : 0;
}
int granite4_kv_pool_mark_written(void* pool, int seq, size_t page_index) {
  return static_cast<PagedKV*>(pool)->mark_written(seq, page_index) ? 1 : 0;
}
int granite4_kv_pool_locate(const void* pool, int seq, size_t token, size_t* out) {
  const auto r = static_cast<const PagedKV*>(pool)->locate(seq, token);
  if (out != nullptr) {
    out[0] = r[0];
    out[1] = r[1];
  }
  return r[0] == SIZE_MAX ? -1 : 0;
}
int granite4_kv_pool_row_table(const void* pool, int seq, size_t n, int32_t* out) {
  return static_cast<const PagedKV*>(pool)->row_table(seq, n, out) ? 0 : -1;
}
void granite4_kv_pool_reset_sequence(void* pool, int seq) {
  static_cast<PagedKV*>(pool)->reset_sequence(seq);
}
void granite4_kv_pool_truncate_sequence(void* pool, int seq, size_t n_tokens) {
  static_cast<PagedKV*>(pool)->truncate_sequence(seq, n_tokens);
}
void granite4_kv_pool_release(void* pool, int seq) { static_cast<PagedKV*>(pool)->release(seq); }
void granite4_kv_pool_clear(void* pool) { static_cast<PagedKV*>(pool)->clear(); }
size_t granite4_kv_pool_block_table(const void* pool, int seq, size_t* out, size_t cap) {
  const auto& bt = static_cast<const PagedKV*>(pool)->block_table(seq);
  for (size_t i = 0; i < bt.size() && i < cap && out != nullptr; ++i) out[i] = bt[i];
  return bt.size();
}
size_t granite4_kv_pool_sequence_tokens(const void* pool, int seq) {
  return static_cast<const PagedKV*>(pool)->sequence_tokens(seq);
}
size_t granite4_kv_pool_ref_count(const void* pool, size_t page_id) {
  return static_cast<const PagedKV*>(pool)->ref_count(page_id);
}
int granite4_kv_pool_page_in_cache(const void* pool, size_t page_id) {
  return static_cast<const PagedKV*>(pool)->page_in_cache(page_id) ? 1 : 0;
}

void* granite4_kv_ctrl_create(size_t layers, size_t kv_heads, size_t head_dim,
                              size_t tokens_per_page, size_t budget_bytes) {
  if (tokens_per_page == 0) return nullptr;
  return new (std::nothrow)
      KvPoolController(config_of(layers, kv_heads, head_dim, tokens_per_page, budget_bytes));
}
void granite4_kv_ctrl_destroy(void* ctrl) { delete static_cast<KvPoolController*>(ctrl); }
size_t granite4_kv_ctrl_stat(const void* ctrl, int which) {
  const auto* c = static_cast<const KvPoolController*>(ctrl);
  switch (which) {
    case GRANITE4_KV_POOL_PAGES: return c->pool_pages();
    case GRANITE4_KV_FREE_PAGES: return c->free_pages();
    case GRANITE4_KV_USED_PAGES: return c->used_pages();
    case GRANITE4_KV_SHARED_PAGES: return c->shared_pages();
    case GRANITE4_KV_CACHED_PAGES: return c->cached_pages();
    case GRANITE4_KV_RETAINED_PAGES: return c->retained_pages();
    case GRANITE4_KV_EVICTED_PAGES: return c->evicted_pages();
    case GRANITE4_KV_TOKENS_PER_PAGE: return c->tokens_per_page();
    default: return SIZE_MAX;
  }
}
int granite4_kv_ctrl_new_slot(void* ctrl) { return static_cast<KvPoolController*>(ctrl)->new_slot(); }
void granite4_kv_ctrl_release_slot(void* ctrl, int slot) {
  static_cast<KvPoolController*>(ctrl)->release_slot(slot);
}
void granite4_kv_ctrl_shutdown(void* ctrl) { static_cast<KvPoolController*>(ctrl)->shutdown(); }
int granite4_kv_ctrl_prefill(void* ctrl, int slot, const uint32_t* prompt, size_t n,
                             size_t* reused) {
  const auto r = static_cast<KvPoolController*>(ctrl)->prefill(slot, ids_of(prompt, n));
  if (reused != nullptr) *reused = r.reused;
  return r.ok ? 0 : -1;
}
void granite4_kv_ctrl_commit(void* ctrl, int slot, const uint32_t* tokens, size_t n) {
  static_cast<KvPoolController*>(ctrl)->commit(slot, ids_of(tokens, n));
}
int granite4_kv_ctrl_open_slot(void* ctrl) { return static_cast<KvPoolController*>(ctrl)->open_slot(); }
int granite4_kv_ctrl_ensure(void* ctrl, int slot, size_t n_tokens) {
  return static_cast<KvPoolController*>(ctrl)->ensure(slot, n_tokens) ? 1 : 0;
}
void granite4_kv_ctrl_trim(void* ctrl, int slot, size_t n_tokens) {
  static_cast<KvPoolController*>(ctrl)->trim(slot, n_tokens);
}
void granite4_kv_ctrl_drop(void* ctrl, int slot) { static_cast<KvPoolController*>(ctrl)->drop(slot); }
size_t granite4_kv_ctrl_pages_missing(const void* ctrl, int slot, size_t n_tokens) {
  return static_cast<const KvPoolController*>(ctrl)->pages_missing(slot, n_tokens);
}
size_t granite4_kv_ctrl_slot_pages(const void* ctrl, int slot) {
  return static_cast<const KvPoolController*>(ctrl)->slot_pages(slot);
}
int granite4_kv_ctrl_row_table(const void* ctrl, int slot, size_t n, int32_t* out) {
  return static_cast<const KvPoolController*>(ctrl)->row_table(slot, n, out) ? 0 : -1;
}
size_t granite4_kv_ctrl_committed(const void* ctrl, int slot) {
  return static_cast<const KvPoolController*>(ctrl)->committed(slot);
}
size_t granite4_kv_ctrl_last_reused(const void* ctrl, int slot) {
  return static_cast<const KvPoolController*>(ctrl)->last_reused(slot);
}

}  // extern "C"
