/*
 * granite4_kv_pool.h - the host page-table controller: the paged KV pool
 * bookkeeping (allocation, ref-counted prefix sharing, LRU retention) that
 * produces the position -> arena-row tables (d_pt) the append and attention
 * kernels of granite4_layerops.h index through.
 *
 * Host-only C++ (no device code). The C++ API keeps the reference's class
 * and method names and meanings (kv_pool.h:58-240, kv_pool_controller.h:
 * 31-128) so engine code written against them compiles unchanged, apart
 * from the layout being built from explicit dimensions instead of the
 * reference's ModelConfig. The C ABI below wraps the same objects for other
 * hosts (Python tests, bindings).
 *
 * Arena rows: page p owns rows [p * tokens_per_page, (p + 1) *
 * tokens_per_page); logical position i of a sequence lives in row
 * block_table[i / B] * B + i % B (B = tokens_per_page), as
 * granite4_row_table computes from a block table.
 */
#ifndef GRANITE4_KV_POOL_H
#define GRANITE4_KV_POOL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
#include <array>
#include <cstdint>
#include <set>
#include <unordered_map>
#include <utility>
#include <vector>

namespace granite4 {

/* One page's byte layout: [token_local][layer][k|v][kv_head][head_dim], one
 * byte per element (kv_pool.h:47-79). */
struct KvLayout {
  std::size_t num_layers = 0;
  std::size_t num_kv_heads = 0;
  std::size_t head_dim = 0;
  std::size_t bytes_per_token = 0;  // 2 * layers * kv_heads * head_dim

  static KvLayout make(std::size_t layers, std::size_t kv_heads, std::size_t head_dim);
  /* Byte offset inside one page, or SIZE_MAX for an index out of range. */
  std::size_t offset(std::size_t tokens_per_page, std::size_t token_local, std::size_t layer,
                     int kv, std::size_t head, std::size_t dim) const;
  std::size_t token_bytes() const { return bytes_per_token; }
};

/* Pool sized from a byte budget: num_pages = floor(budget / page_bytes). */
struct KvPoolConfig {
  KvLayout layout;
  std::size_t tokens_per_page = 16;
  std::size_t budget_bytes = 0;
  std::size_t num_pages = 0;
  std::size_t page_bytes = 0;

  static KvPoolConfig from_budget(const KvLayout& layout, std::size_t tokens_per_page,
                                  std::size_t budget_bytes);
  std::size_t capacity_tokens() const { return num_pages * tokens_per_page; }
  std::size_t total_bytes() const { return num_pages * page_bytes; }
};

/* Paged KV manager (kv_pool.h:109-236): equal-size pages, a block table per
 * sequence, full pages content-addressed by a hash chained over the
 * page-aligned token prefix (verified against the stored tokens on lookup),
 * ref-counted sharing, and pages kept cached at ref count 0 ("retained")
 * until least-recently-used eviction needs them. */
class PagedKV {
 public:
  using Tokens = std::vector<std::uint32_t>;
  explicit PagedKV(KvPoolConfig config);

  int create_sequence();
  std::size_t match_prefix(int seq, const Tokens& tokens);
  bool reserve(int seq, std::size_t token_count, const Tokens& tokens);
  bool mark_written(int seq, std::size_t page_index);
  std::array<std::size_t, 2> locate(int seq, std::size_t token) const;

  std::size_t page_rows() const { return config_.tokens_per_page; }
  std::size_t row_offset(std::size_t page_id) const { return page_id * config_.tokens_per_page; }
  bool row_table(int seq, std::size_t n, int* out) const;

  void reset_sequence(int seq);
  void truncate_sequence(int seq, std::size_t n_tokens);
  void release(int seq);
  void clear();

  const std::vector<std::size_t>& block_table(int seq) const;
  const KvPoolConfig& config() const { return config_; }
  std::size_t pool_pages() const { return config_.num_pages; }
  std::size_t capacity_tokens() const { return config_.capacity_tokens(); }
  std::size_t free_pages() const { return free_.size(); }
  std::size_t used_pages() const { return config_.num_pages - free_.size(); }
  std::size_t shared_pages() const { return shared_; }
  std::size_t cached_pages() const { return cache_.size(); }
  std::size_t evicted_pages() const { return evicted_; }
  std::size_t retained_pages() const { return lru_.size(); }
  std::size_t live_sequences() const { return live_; }
  std::size_t sequence_tokens(int seq) const;
  std::size_t ref_count(std::size_t page_id) const;
  bool page_in_cache(std::size_t page_id) const;

 private:
  struct Page {
    std::vector<std::uint32_t> tokens;  // token ids held (<= tokens_per_page)
    std::uint64_t key = 0;               // cache key while cached
    std::uint64_t tick = 0;              // last use (LRU order)
    int refs = 0;
    bool cached = false;
  };
  struct Seq {
    std::vector<std::size_t> pages;      // block table
    std::vector<std::uint64_t> chain;    // chain[i]: key of the first i full pages
    std::size_t filled = 0;
    bool live = false;
  };

  bool valid(int seq) const;
  void take_ref(std::size_t page);
  void put_ref(std::size_t page);
  void free_page(std::size_t page);
  void uncache(std::size_t page);
  std::size_t evict_lru();
  std::uint64_t prefix_key(Seq& s, std::size_t page_index);

  KvPoolConfig config_;
  std::vector<Page> pages_;
  std::vector<Seq> seqs_;
  std::vector<std::size_t> free_;  // LIFO free list
  std::unordered_map<std::uint64_t, std::size_t> cache_;
  std::set<std::pair<std::uint64_t, std::size_t>> lru_;  // retained pages by tick
  std::uint64_t tick_ = 0;
  std::size_t evicted_ = 0;
  std::size_t shared_ = 0;
  std::size_t live_ = 0;
};

/* Session slots over one PagedKV (kv_pool_controller.h:31-125): prefill
 * adopts the cached prefix and reserves the tail, commit extends and caches
 * newly full pages, and the resident-session calls (open_slot / ensure /
 * trim / drop) manage exclusive pages that never enter the cache. */
class KvPoolController {
 public:
  explicit KvPoolController(KvPoolConfig config);
  ~KvPoolController();
  KvPoolController(const KvPoolController&) = delete;
  KvPoolController& operator=(const KvPoolController&) = delete;

  int new_slot();
  void release_slot(int slot);
  void shutdown();

  struct Prefill {
    int seq = -1;
    std::size_t reused = 0;
    bool ok = false;
  };
  Prefill prefill(int slot, const PagedKV::Tokens& prompt);
  void commit(int slot, const PagedKV::Tokens& all_tokens);

  int open_slot();
  bool ensure(int slot, std::size_t n_tokens);
  void trim(int slot, std::size_t n_tokens);
  void drop(int slot);
  std::size_t pages_missing(int slot, std::size_t n_tokens) const;
  std::size_t slot_pages(int slot) const;

  bool row_table(int slot, std::size_t n, int* out) const;
  std::size_t committed(int slot) const;
  std::size_t last_reused(int slot) const;

  std::size_t max_slots() const { return pool_.pool_pages(); }
  std::size_t pool_pages() const { return pool_.pool_pages(); }
  std::size_t free_pages() const { return pool_.free_pages(); }
  std::size_t used_pages() const { return pool_.used_pages(); }
  std::size_t shared_pages() const { return pool_.shared_pages(); }
  std::size_t cached_pages() const { return pool_.cached_pages(); }
  std::size_t retained_pages() const { return pool_.retained_pages(); }
  std::size_t evicted_pages() const { return pool_.evicted_pages(); }
  std::size_t tokens_per_page() const { return pool_.page_rows(); }

 private:
  struct Slot {
    int seq = -1;
    std::size_t marked = 0;  // leading pages already offered to the cache
    std::size_t reused = 0;
    bool in_use = false;
  };
  const Slot* slot_of(int slot) const;
  void mark_full(Slot& s, std::size_t n_tokens);

  PagedKV pool_;
  std::vector<Slot> slots_;
};

}  // namespace granite4

extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * C ABI over the classes above. Handles are opaque; every call on a NULL or
 * destroyed handle is invalid. Counts are size_t; -1 / 0 failures as noted.
 * ------------------------------------------------------------------------- */

/* Statistic selectors for granite4_kv_pool_stat / granite4_kv_ctrl_stat. */
enum {
  GRANITE4_KV_POOL_PAGES = 0,
  GRANITE4_KV_FREE_PAGES = 1,
  GRANITE4_KV_USED_PAGES = 2,
  GRANITE4_KV_SHARED_PAGES = 3,
  GRANITE4_KV_CACHED_PAGES = 4,
  GRANITE4_KV_RETAINED_PAGES = 5,
  GRANITE4_KV_EVICTED_PAGES = 6,
  GRANITE4_KV_LIVE_SEQUENCES = 7,
  GRANITE4_KV_CAPACITY_TOKENS = 8,
  GRANITE4_KV_PAGE_BYTES = 9,
  GRANITE4_KV_TOKENS_PER_PAGE = 10
};

/* Replaces: KvLayout::offset (kv_pool.cc:40-52); SIZE_MAX when out of range. */
size_t granite4_kv_layout_offset(size_t layers, size_t kv_heads, size_t head_dim,
                                 size_t tokens_per_page, size_t token_local, size_t layer, int kv,
                                 size_t head, size_t dim);

/* Replaces: PagedKV(KvPoolConfig::from_budget(...)) (kv_pool.cc:54-64, 79-83). */
void* granite4_kv_pool_create(size_t layers, size_t kv_heads, size_t head_dim,
                              size_t tokens_per_page, size_t budget_bytes);
void granite4_kv_pool_destroy(void* pool);
size_t granite4_kv_pool_stat(const void* pool, int which);
/* PagedKV methods (kv_pool.h:116-236); bool results as 1 / 0. */
int granite4_kv_pool_create_sequence(void* pool);
size_t granite4_kv_pool_match_prefix(void* pool, int seq, const uint32_t* tokens, size_t n);
int granite4_kv_pool_reserve(void* pool, int seq, size_t token_count, const uint32_t* tokens,
                             size_t n);
int granite4_kv_pool_mark_written(void* pool, int seq, size_t page_index);
/* out[0] = page id, out[1] = token_local; returns 0, or -1 (out = SIZE_MAX). */
int granite4_kv_pool_locate(const void* pool, int seq, size_t token, size_t* out);
/* position -> arena row for positions [0, n); 0, or -1 when n > filled. */
int granite4_kv_pool_row_table(const void* pool, int seq, size_t n, int32_t* out);
void granite4_kv_pool_reset_sequence(void* pool, int seq);
void granite4_kv_pool_truncate_sequence(void* pool, int seq, size_t n_tokens);
void granite4_kv_pool_release(void* pool, int seq);
void granite4_kv_pool_clear(void* pool);
/* Copies up to cap page ids; returns the block table's length. */
size_t granite4_kv_pool_block_table(const void* pool, int seq, size_t* out, size_t cap);
size_t granite4_kv_pool_sequence_tokens(const void* pool, int seq);
size_t granite4_kv_pool_ref_count(const void* pool, size_t page_id);
int granite4_kv_pool_page_in_cache(const void* pool, size_t page_id);

/* Replaces: KvPoolController (kv_pool_controller.h:31-125). */
void* granite4_kv_ctrl_create(size_t layers, size_t kv_heads, size_t head_dim,
                              size_t tokens_per_page, size_t budget_bytes);
void granite4_kv_ctrl_destroy(void* ctrl);
size_t granite4_kv_ctrl_stat(const void* ctrl, int which);
int granite4_kv_ctrl_new_slot(void* ctrl);
void granite4_kv_ctrl_release_slot(void* ctrl, int slot);
void granite4_kv_ctrl_shutdown(void* ctrl);
/* 0 on success (*reused = page-aligned tokens adopted from the cache), -1 when
 * the pool cannot hold the prompt (nothing held afterwards). */
int granite4_kv_ctrl_prefill(void* ctrl, int slot, const uint32_t* prompt, size_t n,
                             size_t* reused);
void granite4_kv_ctrl_commit(void* ctrl, int slot, const uint32_t* tokens, size_t n);
int granite4_kv_ctrl_open_slot(void* ctrl);
int granite4_kv_ctrl_ensure(void* ctrl, int slot, size_t n_tokens);  /* 1 / 0 */
void granite4_kv_ctrl_trim(void* ctrl, int slot, size_t n_tokens);
void granite4_kv_ctrl_drop(void* ctrl, int slot);
size_t granite4_kv_ctrl_pages_missing(const void* ctrl, int slot, size_t n_tokens);
size_t granite4_kv_ctrl_slot_pages(const void* ctrl, int slot);
int granite4_kv_ctrl_row_table(const void* ctrl, int slot, size_t n, int32_t* out);
size_t granite4_kv_ctrl_committed(const void* ctrl, int slot);
size_t granite4_kv_ctrl_last_reused(const void* ctrl, int slot);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* GRANITE4_KV_POOL_H */
