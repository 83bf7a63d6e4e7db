// Host-side compaction planner: page pool, per-group page lists, compacted-span maps and span removal.
//
// Bit-exact with the reference's scheduler/KV-manager bookkeeping (vLLM overlay):
//   free-block FIFO ........ third_party/vllm_overlay/vllm/v1/core/kv_cache_utils.py:157-345
//   page pool .............. third_party/vllm_overlay/vllm/v1/core/block_pool.py:160-176, 295-325, 385-399, 488-550
//   per-group page lists ... third_party/vllm_overlay/vllm/v1/core/single_type_kv_cache_manager.py:66-145, 173-188,
//                            358-452
//   slot allocation ........ third_party/vllm_overlay/vllm/v1/core/kv_cache_manager.py:206-340 (no prefix caching,
//                            no lookahead, no encoder tokens: CompressLM serving disables them)
//   compacted spans ........ third_party/vllm_overlay/vllm/v1/compacted_spans.py:8-68, v1/request.py:263-321
//   span removal ........... third_party/vllm_overlay/vllm/v1/core/sched/scheduler.py:2043-2204
// Pure host code: no HIP call is made from this file.
#include "abridgekv_amd.h"

#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <deque>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace abkv {

struct SpanIndex {
  std::vector<std::pair<int64_t, int64_t>> spans;
  std::vector<int64_t> starts, cumulative, gap_physical, gap_logical;
  int64_t total = 0;

  void rebuild() { rebuild_from(0); }
  // the derived arrays of spans[from:] (entries before `from` are unchanged by an insertion or merge at `from`)
  void rebuild_from(size_t from) {
    const size_t n = spans.size();
    starts.resize(n);
    cumulative.resize(n);
    gap_physical.resize(n + 1);
    gap_logical.resize(n + 1);
    gap_physical[0] = 0;
    gap_logical[0] = 0;
    total = from > 0 ? cumulative[from - 1] : 0;
    for (size_t k = from; k < n; ++k) {
      starts[k] = spans[k].first;
      total += spans[k].second - spans[k].first;
      cumulative[k] = total;
      gap_physical[k + 1] = spans[k].second - total;
      gap_logical[k + 1] = spans[k].second;
    }
  }
  // some span overlaps [start, end) (the spans are sorted and disjoint)
  bool overlaps(int64_t start, int64_t end) const {
    long i = idx_le(end - 1);                     // the last span starting before end
    return i >= 0 && spans[(size_t)i].second > start;
  }
  // bisect_right(starts, pos) - 1
  long idx_le(int64_t pos) const {
    return (long)(std::upper_bound(starts.begin(), starts.end(), pos) - starts.begin()) - 1;
  }
  bool is_active(int64_t pos) const {
    if (starts.empty()) return true;
    long i = idx_le(pos);
    if (i < 0) return true;
    return pos >= spans[i].second;
  }
  int64_t l2p(int64_t pos) const {
    if (starts.empty()) return pos;
    long i = idx_le(pos);
    if (i < 0) return pos;
    if (pos >= spans[i].second) return pos - cumulative[i];
    int64_t prev = i > 0 ? cumulative[i - 1] : 0;
    return pos - prev - (pos - starts[i]);
  }
  int64_t p2l(int64_t phys) const {
    long i = (long)(std::upper_bound(gap_physical.begin(), gap_physical.end(), phys) - gap_physical.begin()) - 1;
    return gap_logical[i] + (phys - gap_physical[i]);
  }
  // spans = merge(spans + [span]): the list is already sorted and merged, so the new span goes to its sorted place
  // and can only merge with the span before it and the spans after it that it reaches (no temporary list)
  void add_merged(std::pair<int64_t, int64_t> span) {
    size_t i = (size_t)(std::lower_bound(spans.begin(), spans.end(), span) - spans.begin());
    spans.insert(spans.begin() + (long)i, span);
    if (i > 0 && spans[i].first <= spans[i - 1].second) {
      spans[i - 1].second = std::max(spans[i - 1].second, spans[i].second);
      spans.erase(spans.begin() + (long)i);
      --i;
    }
    size_t j = i + 1;
    while (j < spans.size() && spans[j].first <= spans[i].second) spans[i].second = std::max(spans[i].second, spans[j++].second);
    spans.erase(spans.begin() + (long)(i + 1), spans.begin() + (long)j);
    rebuild_from(i);
  }
};

struct Op {
  int32_t src_block, src_off, dst_block, dst_off;
};

// One span removal applied to one group of one request during the current step (physical coordinates of the
// layout the removal saw).
struct Removal {
  int64_t start, end, active;
};

struct GroupStep {
  std::vector<std::vector<Op>> batches;   // reference-format ordered op batches
  // pages blocks_lo .. of the page list before the step's first removal: every row a step's moves read or write lies
  // at or after its lowest removal start, and no removal or allocation changes a page below its own start's page, so
  // the pages below the first removal's are copied in only when a later removal of the step starts lower
  std::vector<int32_t> blocks_before;
  int64_t blocks_lo = 0;
  std::vector<Removal> removals;
  bool stale = false;                     // a removal followed an allocation that followed a removal (no take)
  // the state of a step with no removal; the vectors keep their capacity for the next step
  void reset() {
    batches.clear();
    blocks_before.clear();
    blocks_lo = 0;
    removals.clear();
    stale = false;
  }
};

// One group's part of a span removal, validated before any group is changed.
struct SpanPlan {
  int g;
  int64_t ps, pe, active;
};

struct Request {
  int64_t num_computed = 0;
  std::vector<SpanIndex> spans;           // per group
  std::vector<std::vector<int32_t>> blocks;  // per group
  std::vector<GroupStep> step;            // per group, cleared by take_step_outputs
  bool has_trunc = false;
  std::vector<int32_t> trunc;
  bool alloc_after_removal = false;       // an allocation happened while removals were pending
};

struct Planner {
  int num_blocks = 0, num_groups = 0, block_size = 16;
  int64_t max_model_len = 0;
  int32_t null_block = 0;
  std::vector<int32_t> ref_cnt;
  std::deque<int32_t> free_q;
  std::unordered_map<int64_t, Request> reqs;
  std::vector<int64_t> pending_order;     // rids with pending ops, first-insertion order
  std::vector<int64_t> trunc_order;       // rids with a truncation record, first-insertion order
  std::string last_error;
  bool op_rows = true;                    // build the reference-format op batches (off: fused moves only)
  // scratch of abkv_planner_mask_token_span, kept between calls
  std::vector<int> mts_targets;
  std::vector<SpanPlan> mts_plans;
  std::vector<int32_t> mts_free;
  // scratch of abkv_planner_take_moves_packed, kept between steps
  std::vector<int64_t> mv_origin;
  std::vector<uint8_t> mv_chained;
  int bs_shift = -1;                      // log2(block_size) when it is a power of two

  // slot position -> (page index, offset) without a division when the page size is a power of two
  int64_t page_of(int64_t pos) const { return bs_shift >= 0 ? pos >> bs_shift : pos / block_size; }
  int32_t off_of(int64_t pos) const {
    return (int32_t)(bs_shift >= 0 ? pos & ((int64_t)block_size - 1) : pos % block_size);
  }

  int64_t cdiv(int64_t a, int64_t b) const { return (a + b - 1) / b; }

  bool get_new_blocks(int64_t n, std::vector<int32_t>& out) {
    if (n > (int64_t)free_q.size()) {
      last_error = "Cannot get " + std::to_string(n) + " free blocks from the pool";
      return false;
    }
    for (int64_t i = 0; i < n; ++i) {
      int32_t b = free_q.front();
      free_q.pop_front();
      ref_cnt[b] += 1;
      out.push_back(b);
    }
    return true;
  }

  void free_blocks(const std::vector<int32_t>& ordered) {
    for (int32_t b : ordered) ref_cnt[b] -= 1;
    for (int32_t b : ordered)
      if (ref_cnt[b] == 0 && b != null_block) free_q.push_back(b);
  }
};

static void note_order(std::vector<int64_t>& order, int64_t rid) {
  if (std::find(order.begin(), order.end(), rid) == order.end()) order.push_back(rid);
}

}  // namespace abkv

using abkv::Planner;
using abkv::Request;

extern "C" {

// Error codes of the planner entry points.

void* abkv_planner_create(int num_blocks, int num_groups, int block_size, const int32_t* free_order,
                          int64_t max_model_len) {
  if (num_blocks < 2 || num_groups < 1 || block_size < 1) return nullptr;
  Planner* p = new Planner();
  p->num_blocks = num_blocks;
  p->num_groups = num_groups;
  p->block_size = block_size;
  if ((block_size & (block_size - 1)) == 0)
    while ((1 << (p->bs_shift + 1)) <= block_size) ++p->bs_shift;
  p->max_model_len = max_model_len > 0 ? max_model_len : ((int64_t)1 << 40);
  p->ref_cnt.assign(num_blocks, 0);
  p->null_block = 0;  // the queue starts in id order and its head (page 0) becomes the null block
  if (free_order != nullptr) {
    std::vector<char> seen(num_blocks, 0);
    for (int i = 0; i < num_blocks - 1; ++i) {
      int32_t b = free_order[i];
      if (b < 1 || b >= num_blocks || seen[b]) {
        delete p;
        return nullptr;
      }
      seen[b] = 1;
      p->free_q.push_back(b);
    }
  } else {
    for (int32_t b = 1; b < num_blocks; ++b) p->free_q.push_back(b);
  }
  return p;
}

void abkv_planner_destroy(void* h) { delete static_cast<Planner*>(h); }

// Build (1, the default) or skip (0) the reference-format op batches. With 0 the planner's bookkeeping (spans, page
// lists, truncations, the free queue) is unchanged and the fused moves are still emitted; take_step_outputs then
// returns no op rows. For callers that execute the fused moves only.
int abkv_planner_set_op_rows(void* h, int enabled) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  p->op_rows = enabled != 0;
  return ABKV_OK;
}

const char* abkv_planner_last_error(void* h) { return h ? static_cast<Planner*>(h)->last_error.c_str() : ""; }

int abkv_planner_add_request(void* h, int64_t rid) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  Request& r = p->reqs[rid];
  r.num_computed = 0;
  r.spans.assign(p->num_groups, abkv::SpanIndex());
  for (auto& s : r.spans) s.rebuild();
  r.blocks.assign(p->num_groups, {});
  r.step.assign(p->num_groups, {});
  r.has_trunc = false;
  return ABKV_OK;
}

static Request* find_req(Planner* p, int64_t rid) {
  auto it = p->reqs.find(rid);
  return it == p->reqs.end() ? nullptr : &it->second;
}

// coordinator.free: every group frees its pages in reverse order (single_type_kv_cache_manager.py:173-188).
int abkv_planner_free_request(void* h, int64_t rid) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  Request* r = find_req(p, rid);
  if (!r) return ABKV_ERR_NO_REQUEST;
  for (int g = 0; g < p->num_groups; ++g) {
    std::vector<int32_t> rev(r->blocks[g].rbegin(), r->blocks[g].rend());
    p->free_blocks(rev);
  }
  p->reqs.erase(rid);
  p->pending_order.erase(std::remove(p->pending_order.begin(), p->pending_order.end(), rid), p->pending_order.end());
  p->trunc_order.erase(std::remove(p->trunc_order.begin(), p->trunc_order.end(), rid), p->trunc_order.end());
  return ABKV_OK;
}

int abkv_planner_set_num_computed(void* h, int64_t rid, int64_t n) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  Request* r = find_req(p, rid);
  if (!r) return ABKV_ERR_NO_REQUEST;
  r->num_computed = n;
  return ABKV_OK;
}

int64_t abkv_planner_get_num_computed(void* h, int64_t rid) {
  Planner* p = static_cast<Planner*>(h);
  Request* r = p ? find_req(p, rid) : nullptr;
  return r ? r->num_computed : -1;
}

// Returns 1 when pages were (or did not need to be) allocated, 0 when the pool cannot cover the request (the
// reference returns None and allocates nothing), negative on error.
int abkv_planner_allocate_slots(void* h, int64_t rid, int64_t num_new_tokens) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  Request* r = find_req(p, rid);
  if (!r) return ABKV_ERR_NO_REQUEST;
  if (num_new_tokens == 0) {
    p->last_error = "num_new_tokens must be greater than 0";
    return ABKV_ERR_ARG;
  }
  const int64_t need = std::min(r->num_computed + num_new_tokens, p->max_model_len);
  int64_t total = 0;
  for (int g = 0; g < p->num_groups; ++g)
    total += p->cdiv(need - r->spans[g].total, p->block_size) - (int64_t)r->blocks[g].size();
  if (total > (int64_t)p->free_q.size()) return 0;
  for (auto& st : r->step)
    if (!st.removals.empty()) r->alloc_after_removal = true;
  for (int g = 0; g < p->num_groups; ++g) {
    const int64_t num_new = p->cdiv(need - r->spans[g].total, p->block_size) - (int64_t)r->blocks[g].size();
    if (num_new <= 0) continue;
    if (!p->get_new_blocks(num_new, r->blocks[g])) return ABKV_ERR_POOL;
  }
  return 1;
}

// Scheduler.mask_token_span. groups == nullptr (or n_groups < 0) targets every group. Returns ABKV_OK on success
// (tokens_removed / blocks_freed filled), ABKV_ERR_SPAN with last_error holding the reference's error message.
int abkv_planner_mask_token_span(void* h, int64_t rid, int64_t start, int64_t end, const int32_t* groups,
                                 int n_groups, int64_t* tokens_removed, int64_t* blocks_freed) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  if (tokens_removed) *tokens_removed = 0;
  if (blocks_freed) *blocks_freed = 0;
  Request* r = find_req(p, rid);
  if (!r) {
    p->last_error = "Request " + std::to_string(rid) + " not found";
    return ABKV_ERR_SPAN;
  }
  if (start < 0 || end <= start) {
    p->last_error = "Invalid span: must have 0 <= start < end";
    return ABKV_ERR_SPAN;
  }
  if (end > r->num_computed) {
    p->last_error = "end_position (" + std::to_string(end) + ") exceeds computed tokens (" +
                    std::to_string(r->num_computed) + ")";
    return ABKV_ERR_SPAN;
  }
  const int64_t masked = end - start;
  const int G = p->num_groups;
  std::vector<int>& targets = p->mts_targets;
  targets.clear();
  if (groups == nullptr || n_groups < 0) {
    for (int g = 0; g < G; ++g) targets.push_back(g);
  } else {
    for (int i = 0; i < n_groups; ++i) targets.push_back(groups[i]);
    std::sort(targets.begin(), targets.end());
    targets.erase(std::unique(targets.begin(), targets.end()), targets.end());
  }
  std::vector<abkv::SpanPlan>& plans = p->mts_plans;
  plans.clear();
  for (int g : targets) {
    if (g < 0 || g >= G) {
      p->last_error = "KV cache group " + std::to_string(g) + " out of range";
      return ABKV_ERR_SPAN;
    }
    if (r->spans[g].overlaps(start, end)) {
      p->last_error = "Cannot compact an already-removed token span (group " + std::to_string(g) + ")";
      return ABKV_ERR_SPAN;
    }
    const int64_t ps = r->spans[g].l2p(start), pe = r->spans[g].l2p(end);
    if (pe - ps != masked) {
      p->last_error = "Logical span does not map to one active physical span (group " + std::to_string(g) + ")";
      return ABKV_ERR_SPAN;
    }
    const int64_t active = r->num_computed - r->spans[g].total;
    if (active == masked) {
      p->last_error = "Cannot compact: all tokens would be removed";
      return ABKV_ERR_SPAN;
    }
    plans.push_back({g, ps, pe, active});
  }
  int64_t total_freed = 0;
  const int bs = p->block_size;
  for (auto& pl : plans) {
    std::vector<int32_t>& blocks = r->blocks[pl.g];
    abkv::GroupStep& st = r->step[pl.g];
    if (!(0 <= pl.ps && pl.ps < pl.pe && pl.pe <= pl.active)) {
      p->last_error = "Invalid physical compaction span";
      return ABKV_ERR_SPAN;
    }
    if (!blocks.empty()) {
      const int64_t lo_page = p->page_of(pl.ps);
      if (st.removals.empty()) {
        st.blocks_lo = lo_page;
        st.blocks_before.assign(blocks.begin() + lo_page, blocks.end());
      } else {
        if (r->alloc_after_removal) st.stale = true;
        if (lo_page < st.blocks_lo) {
          st.blocks_before.insert(st.blocks_before.begin(), blocks.begin() + lo_page, blocks.begin() + st.blocks_lo);
          st.blocks_lo = lo_page;
        }
      }
      st.removals.push_back({pl.ps, pl.pe, pl.active});
      const int64_t removed = pl.pe - pl.ps;
      std::vector<abkv::Op> ops;
      if (p->op_rows) {
        ops.reserve((size_t)(pl.active - pl.pe));
        for (int64_t src = pl.pe; src < pl.active; ++src) {
          const int64_t dst = src - removed;
          ops.push_back({blocks[p->page_of(src)], p->off_of(src), blocks[p->page_of(dst)], p->off_of(dst)});
        }
      }
      // _truncate_compacted_blocks
      const int64_t needed = (pl.active - removed + bs - 1) / bs;
      std::vector<int32_t>& to_free = p->mts_free;
      to_free.clear();
      for (int64_t i = needed; i < (int64_t)blocks.size(); ++i) {
        if (blocks[i] != p->null_block) {
          to_free.push_back(blocks[i]);
          blocks[i] = p->null_block;
          ++total_freed;
        }
      }
      if ((int64_t)blocks.size() > needed) blocks.resize((size_t)needed);
      if (!to_free.empty()) {
        std::reverse(to_free.begin(), to_free.end());
        p->free_blocks(to_free);
      }
      if (!ops.empty()) {
        st.batches.push_back(std::move(ops));
        abkv::note_order(p->pending_order, rid);
      }
    }
    r->spans[pl.g].add_merged({start, end});
  }
  r->has_trunc = true;
  r->trunc.resize(G);
  for (int g = 0; g < G; ++g) r->trunc[g] = (int32_t)r->blocks[g].size();
  abkv::note_order(p->trunc_order, rid);
  if (tokens_removed) *tokens_removed = masked;
  if (blocks_freed) *blocks_freed = total_freed;
  return ABKV_OK;
}

// Sizes of the pending step outputs: reference-format op rows, truncation rows and fused move rows.
int abkv_planner_pending_sizes(void* h, int64_t* n_op_rows, int64_t* n_trunc_rows, int64_t* n_fused_rows) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  int64_t ops = 0, fused = 0;
  for (int64_t rid : p->pending_order) {
    Request* r = find_req(p, rid);
    for (auto& st : r->step)
      for (auto& b : st.batches) ops += (int64_t)b.size();
  }
  for (auto& kv : p->reqs)
    for (auto& st : kv.second.step)
      if (!st.removals.empty()) {
        const int64_t lo = std::min_element(st.removals.begin(), st.removals.end(),
                                            [](const abkv::Removal& a, const abkv::Removal& b) {
                                              return a.start < b.start;
                                            })->start;
        fused += st.removals.front().active - lo;   // upper bound
      }
  if (n_op_rows) *n_op_rows = ops;
  if (n_trunc_rows) *n_trunc_rows = (int64_t)p->trunc_order.size();
  if (n_fused_rows) *n_fused_rows = fused;
  return ABKV_OK;
}

// Emit and clear the step outputs.
//  op_rows    [n_op_rows, 7]  = (rid, group, batch, src_block, src_off, dst_block, dst_off), in the order the
//             reference's SchedulerOutput.kv_copy_operations dict iterates (request first-insertion order, group,
//             batch, op).
//  trunc_rows [n_trunc_rows, 1 + G] = (rid, pages kept per group), pending_block_table_truncations order.
//  fused_rows [n_fused, 6] = (rid, group, src_block, src_off, dst_block, dst_off): all of a step's removals of one
//             (request, group) composed into one monotone move list (increasing source, dst < src), restricted to
//             rows that survive the step; rows the reference moves and then truncates are not moved.
// Any output pointer may be null to skip it. Returns ABKV_ERR_CAPACITY if a capacity is too small (nothing
// cleared).
int abkv_planner_take_step_outputs(void* h, int64_t* op_rows, int64_t op_cap, int64_t* n_ops, int64_t* trunc_rows,
                                   int64_t trunc_cap, int64_t* n_trunc, int64_t* fused_rows, int64_t fused_cap,
                                   int64_t* n_fused) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  int64_t need_ops = 0, need_trunc = 0, need_fused = 0;
  abkv_planner_pending_sizes(h, &need_ops, &need_trunc, &need_fused);
  for (int64_t rid : p->trunc_order)
    for (auto& st : find_req(p, rid)->step)
      if (st.stale) {
        p->last_error = "span removals of one step were interleaved with an allocation: take the step outputs "
                        "once per scheduler step";
        return ABKV_ERR_ARG;
      }
  if ((op_rows && need_ops > op_cap) || (trunc_rows && need_trunc > trunc_cap)) return ABKV_ERR_CAPACITY;
  const int G = p->num_groups;
  int64_t k = 0;
  if (op_rows) {
    for (int64_t rid : p->pending_order) {
      Request* r = find_req(p, rid);
      for (int g = 0; g < G; ++g) {
        auto& st = r->step[g];
        for (size_t b = 0; b < st.batches.size(); ++b)
          for (auto& op : st.batches[b]) {
            int64_t* row = op_rows + 7 * k++;
            row[0] = rid;
            row[1] = g;
            row[2] = (int64_t)b;
            row[3] = op.src_block;
            row[4] = op.src_off;
            row[5] = op.dst_block;
            row[6] = op.dst_off;
          }
      }
    }
  }
  if (n_ops) *n_ops = op_rows ? k : need_ops;
  int64_t t = 0;
  if (trunc_rows) {
    for (int64_t rid : p->trunc_order) {
      Request* r = find_req(p, rid);
      int64_t* row = trunc_rows + (1 + G) * t++;
      row[0] = rid;
      for (int g = 0; g < G; ++g) row[1 + g] = r->trunc[g];
    }
  }
  if (n_trunc) *n_trunc = trunc_rows ? t : need_trunc;
  // Fused moves in request first-insertion order of the truncation records (every compacting request has one).
  int64_t f = 0;
  for (int64_t rid : p->trunc_order) {
    Request* r = find_req(p, rid);
    for (int g = 0; g < G; ++g) {
      auto& st = r->step[g];
      if (st.removals.empty()) continue;
      int64_t lo = st.removals[0].start;
      for (auto& rm : st.removals) lo = std::min(lo, rm.start);
      const int64_t active0 = st.removals.front().active;
      std::vector<int64_t> origin;
      origin.reserve((size_t)(active0 - lo));
      for (int64_t s = lo; s < active0; ++s) origin.push_back(s);
      for (auto& rm : st.removals)
        origin.erase(origin.begin() + (rm.start - lo), origin.begin() + (rm.end - lo));
      for (size_t i = 0; i < origin.size(); ++i) {
        const int64_t dst = lo + (int64_t)i, src = origin[i];
        if (src == dst) continue;
        if (fused_rows) {
          if (f >= fused_cap) return ABKV_ERR_CAPACITY;
          int64_t* row = fused_rows + 6 * f;
          row[0] = rid;
          row[1] = g;
          row[2] = st.blocks_before[p->page_of(src) - st.blocks_lo];
          row[3] = p->off_of(src);
          row[4] = st.blocks_before[p->page_of(dst) - st.blocks_lo];
          row[5] = p->off_of(dst);
        }
        ++f;
      }
    }
  }
  if (n_fused) *n_fused = f;
  for (auto& kv : p->reqs) {
    for (auto& st : kv.second.step) st.reset();
    kv.second.has_trunc = false;
    kv.second.alloc_after_removal = false;
  }
  p->pending_order.clear();
  p->trunc_order.clear();
  return ABKV_OK;
}

// The step's outputs for a caller that executes fused moves: the truncation rows of abkv_planner_take_step_outputs
// and, instead of fused rows, the device move lists abkv_moves_pack would build from them, written directly (the
// dependency of a run is found from physical positions: the run's destinations are exactly [lo, lo + n), so op i is
// on an edge when origin[i] - lo names a moved op). The step is cleared as by take_step_outputs (op batches, if
// built, are dropped). out_cap >= 5 * (the fused bound of abkv_planner_pending_sizes) + 4 * num_groups. Returns the
// int32 elements written to `out` (index [num_groups, 5] as abkv_moves_pack), ABKV_ERR_CAPACITY or ABKV_ERR_ARG.
int64_t abkv_planner_take_moves_packed(void* h, int64_t* trunc_rows, int64_t trunc_cap, int64_t* n_trunc,
                                       int32_t* out, int64_t out_cap, int64_t* index) {
  Planner* p = static_cast<Planner*>(h);
  if (!p || !out || !index) return ABKV_ERR_ARG;
  int64_t need_ops = 0, need_trunc = 0, need_fused = 0;
  abkv_planner_pending_sizes(h, &need_ops, &need_trunc, &need_fused);
  for (int64_t rid : p->trunc_order)
    for (auto& st : find_req(p, rid)->step)
      if (st.stale) {
        p->last_error = "span removals of one step were interleaved with an allocation: take the step outputs "
                        "once per scheduler step";
        return ABKV_ERR_ARG;
      }
  const int G = p->num_groups;
  if ((trunc_rows && need_trunc > trunc_cap) || out_cap < 5 * need_fused + 4 * (int64_t)G) return ABKV_ERR_CAPACITY;
  int64_t t = 0;
  if (trunc_rows) {
    for (int64_t rid : p->trunc_order) {
      Request* r = find_req(p, rid);
      int64_t* row = trunc_rows + (1 + G) * t++;
      row[0] = rid;
      for (int g = 0; g < G; ++g) row[1 + g] = r->trunc[g];
    }
  }
  if (n_trunc) *n_trunc = trunc_rows ? t : need_trunc;
  // Pass 1: every run's surviving rows (origin) and which of them lie on a dependency edge, into flat scratch kept
  // between steps; per group counts. Pass 2 writes each op once, at its final place in `out`.
  struct RunInfo {
    int g;
    int64_t lo, n, at;                                    // at: the run's first row in the flat scratch
    const int32_t* blocks;                                // pages blocks_lo ..
    int64_t blocks_lo;
    bool any;
  };
  std::vector<RunInfo> runs;
  std::vector<int64_t> n_ord_g((size_t)G, 0), n_free_g((size_t)G, 0), n_seg_g((size_t)G, 0);
  std::vector<int64_t>& origin = p->mv_origin;
  std::vector<uint8_t>& chained = p->mv_chained;
  int64_t total = 0;
  for (int64_t rid : p->trunc_order) {
    Request* r = find_req(p, rid);
    for (int g = 0; g < G; ++g) {
      const auto& st = r->step[g];
      if (st.removals.empty()) continue;
      int64_t lo = st.removals[0].start, removed = 0;
      for (auto& rm : st.removals) {
        lo = std::min(lo, rm.start);
        removed += rm.end - rm.start;
      }
      runs.push_back({g, lo, std::max<int64_t>(st.removals.front().active - lo - removed, 0), total,
                      st.blocks_before.data(), st.blocks_lo, false});
      total += runs.back().n;
    }
  }
  if ((int64_t)origin.size() < total) origin.resize((size_t)total);
  if ((int64_t)chained.size() < total) chained.resize((size_t)total);
  size_t ri = 0;
  for (int64_t rid : p->trunc_order) {
    Request* r = find_req(p, rid);
    for (int g = 0; g < G; ++g) {
      const auto& st = r->step[g];
      if (st.removals.empty()) continue;
      RunInfo& run = runs[ri++];
      const int64_t lo = run.lo, n = run.n;
      int64_t* org = origin.data() + run.at;
      uint8_t* ch = chained.data() + run.at;
      // final row i came from position lo + x, x found by undoing the removals last to first (each removal's span
      // is in the coordinates the earlier ones left)
      for (int64_t i = 0; i < n; ++i) {
        int64_t x = i;
        for (size_t k = st.removals.size(); k-- > 0;)
          if (x >= st.removals[k].start - lo) x += st.removals[k].end - st.removals[k].start;
        org[i] = lo + x;
        ch[i] = 0;
      }
      // op i (row i, moved when org[i] != lo + i) reads org[i], the destination of op j = org[i] - lo when that row
      // moves too: both lie on an edge
      int64_t n_moved = 0, n_ch = 0;
      for (int64_t i = 0; i < n; ++i) {
        if (org[i] == lo + i) continue;
        ++n_moved;
        const int64_t j = org[i] - lo;
        if (j < n && org[j] != lo + j) {
          n_ch += !ch[i] + !ch[j];
          ch[i] = ch[j] = 1;
        }
      }
      run.any = n_ch > 0;
      n_ord_g[(size_t)g] += n_ch;
      n_free_g[(size_t)g] += n_moved - n_ch;
      n_seg_g[(size_t)g] += run.any;
    }
  }
  // layout, then pass 2
  std::vector<int32_t*> ord_c((size_t)G), fre_c((size_t)G), seg_c((size_t)G);
  int64_t at = 0;
  for (int g = 0; g < G; ++g) {
    const int64_t n_ord = n_ord_g[(size_t)g], n_free = n_free_g[(size_t)g], n_seg = n_seg_g[(size_t)g];
    int32_t* ops = out + at;
    int32_t* offs = ops + 4 * (n_ord + n_free);
    ord_c[(size_t)g] = ops;
    fre_c[(size_t)g] = ops + 4 * n_ord;
    offs[0] = 0;
    for (int64_t k2 = n_seg + 1; k2 < ((n_seg + 1 + 3) & ~(int64_t)3); ++k2) offs[k2] = 0;   // alignment padding
    seg_c[(size_t)g] = offs + 1;
    int64_t* ix = index + 5 * g;
    ix[0] = at;
    ix[1] = n_ord + n_free;
    ix[2] = at + 4 * (n_ord + n_free);
    ix[3] = n_seg;
    ix[4] = n_free;
    at += 4 * (n_ord + n_free) + ((n_seg + 1 + 3) & ~(int64_t)3);
  }
  for (const RunInfo& run : runs) {
    const int g = run.g;
    const int64_t* org = origin.data() + run.at;
    const uint8_t* ch = chained.data() + run.at;
    int32_t* vo = ord_c[(size_t)g];
    int32_t* vf = fre_c[(size_t)g];
    for (int64_t i = 0; i < run.n; ++i) {
      const int64_t src = org[i], dst = run.lo + i;
      if (src == dst) continue;
      int32_t* d = ch[i] ? vo : vf;
      d[0] = run.blocks[p->page_of(src) - run.blocks_lo];
      d[1] = p->off_of(src);
      d[2] = run.blocks[p->page_of(dst) - run.blocks_lo];
      d[3] = p->off_of(dst);
      if (ch[i]) vo += 4;
      else vf += 4;
    }
    if (run.any) *seg_c[(size_t)g]++ = (int32_t)((vo - (out + index[5 * g])) / 4);
    ord_c[(size_t)g] = vo;
    fre_c[(size_t)g] = vf;
  }
  for (auto& kv : p->reqs) {
    for (auto& st : kv.second.step) st.reset();
    kv.second.has_trunc = false;
    kv.second.alloc_after_removal = false;
  }
  p->pending_order.clear();
  p->trunc_order.clear();
  return at;
}

namespace {

// Run descriptor of abkv_planner_take_move_runs (int32 fields; layout shared with moves_expand_kernel).
constexpr int kRunRemovalsMax = 8;
constexpr int kRunFields = 14 + 2 * kRunRemovalsMax;

// The row map of one (request, group) run in closed form. Final row i (relative to lo) came from lo + f(i): undoing
// the removals last to first adds removal k's length exactly from the first final row whose partially undone
// position reaches the removal's start, so f(i) = i + c[J(i)] with tau sorted ascending, c the running sums of the
// lengths in that order and J(i) the number of thresholds <= i.
struct RowMap {
  int m = 0;
  int64_t tau[kRunRemovalsMax], c[kRunRemovalsMax];
  int64_t f(int64_t x) const {
    int64_t add = 0;
    for (int j = 0; j < m; ++j) add = x >= tau[j] ? c[j] : add;
    return x + add;
  }
  // smallest x >= 0 with f(x) >= y
  int64_t inv(int64_t y) const {
    for (int j = 0; j <= m; ++j) {
      const int64_t lo = j == 0 ? 0 : tau[j - 1], add = j == 0 ? 0 : c[j - 1];
      const int64_t x = std::max(lo, y - add);
      if (j == m || x < tau[j]) return x;
    }
    return y;
  }
};

// Thresholds of the removals of one run (start, len in the coordinates the earlier removals left, relative to lo):
// false when there are more than kRunRemovalsMax non-empty removals.
bool build_row_map(const std::vector<abkv::Removal>& rm, int64_t lo, RowMap& out) {
  int64_t tau[kRunRemovalsMax], len[kRunRemovalsMax];
  int m = 0;
  for (size_t k = rm.size(); k-- > 0;) {               // last removal first: its threshold is its own start
    const int64_t L = rm[k].end - rm[k].start;
    if (L <= 0) continue;
    if (m == kRunRemovalsMax) return false;
    // smallest x with x + (lengths of the later removals whose thresholds are <= x) >= start - lo
    RowMap later;
    later.m = m;
    int order[kRunRemovalsMax];
    for (int j = 0; j < m; ++j) order[j] = j;
    std::sort(order, order + m, [&](int a, int b) { return tau[a] < tau[b]; });
    int64_t run = 0;
    for (int j = 0; j < m; ++j) {
      later.tau[j] = tau[order[j]];
      run += len[order[j]];
      later.c[j] = run;
    }
    tau[m] = later.inv(rm[k].start - lo);
    len[m] = L;
    ++m;
  }
  int order[kRunRemovalsMax];
  for (int j = 0; j < m; ++j) order[j] = j;
  std::stable_sort(order, order + m, [&](int a, int b) { return tau[a] < tau[b]; });
  out.m = m;
  int64_t run = 0;
  for (int j = 0; j < m; ++j) {
    out.tau[j] = tau[order[j]];
    run += len[order[j]];
    out.c[j] = run;
  }
  return true;
}

}  // namespace

// Sizes of abkv_planner_take_move_runs for the pending step: runs (records) and pages (int32) it will write.
int abkv_planner_pending_run_sizes(void* h, int64_t* n_runs, int64_t* n_pages) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  int64_t runs = 0, pages = 0;
  for (int64_t rid : p->trunc_order) {
    Request* r = find_req(p, rid);
    for (auto& st : r->step) {
      if (st.removals.empty()) continue;
      ++runs;
      int64_t lo = st.removals[0].start;
      for (auto& rm : st.removals) lo = std::min(lo, rm.start);
      pages += p->page_of(std::max<int64_t>(st.removals.front().active - 1, lo)) - p->page_of(lo) + 1;
    }
  }
  if (n_runs) *n_runs = runs;
  if (n_pages) *n_pages = pages;
  return ABKV_OK;
}

// The step's fused moves as run descriptors that abkv_moves_expand turns into exactly the move lists
// abkv_planner_take_moves_packed writes (same index, same element order), so the host does O(runs + pages) work and
// the device the O(rows) part. Per (request, group) run with moved rows, one record of kRunFields int32:
//   0 n (rows of the run), 1 lo_w (the run's first row within its page window), 2 pages_at, 3 ord_at and 4 free_at
//   (int32 element positions in `out` of the run's first ordered / independent op), 5 n_chained, 6 n_free,
//   7 seg_at (-1: the run has no ordered op) and 8 its segment offset, 9 m, 10 t_star (first moved row),
//   11 a_end (rows [t_star, a_end) read a row the run also writes), 12 pages in the window, 13 unused, 14.. tau[m],
//   then c[m] at 14 + kRunRemovalsMax
// pages: each run's page window (the pages of rows lo .. the run's last source row). groups [num_groups, 4] =
// (offs_at, n_segments, end of the section's padding, 0) for the offsets' first entry and padding. index as
// abkv_planner_take_moves_packed. sizes = (records written, pages written, int32 elements of `out`). Clears the step as
// take_moves_packed does. ABKV_ERR_CAPACITY (nothing cleared) or ABKV_ERR_ARG (page size not a power of two, more
// than kRunRemovalsMax removals in one run, or a step interleaved with an allocation).
int abkv_planner_take_move_runs(void* h, int64_t* trunc_rows, int64_t trunc_cap, int64_t* n_trunc, int32_t* runs,
                                int64_t runs_cap, int32_t* pages, int64_t pages_cap, int32_t* groups, int64_t* index,
                                int64_t* sizes) {
  Planner* p = static_cast<Planner*>(h);
  if (!p || !runs || !pages || !groups || !index || !sizes) return ABKV_ERR_ARG;
  if (p->bs_shift < 0) {
    p->last_error = "move runs need a power-of-two page size";
    return ABKV_ERR_ARG;
  }
  for (int64_t rid : p->trunc_order)
    for (auto& st : find_req(p, rid)->step)
      if (st.stale) {
        p->last_error = "span removals of one step were interleaved with an allocation: take the step outputs "
                        "once per scheduler step";
        return ABKV_ERR_ARG;
      }
  int64_t need_runs = 0, need_pages = 0, need_trunc = (int64_t)p->trunc_order.size();
  abkv_planner_pending_run_sizes(h, &need_runs, &need_pages);
  if ((trunc_rows && need_trunc > trunc_cap) || need_runs > runs_cap || need_pages > pages_cap)
    return ABKV_ERR_CAPACITY;
  const int G = p->num_groups;
  struct RunInfo {
    int g;
    int64_t lo, n, n_ch, n_moved, t_star, a_end;
    RowMap map;
    const std::vector<int32_t>* blocks;                   // pages blocks_lo ..
    int64_t blocks_lo, win_lo, win_n;
  };
  std::vector<RunInfo> infos;
  infos.reserve((size_t)need_runs);
  std::vector<int64_t> n_ord_g((size_t)G, 0), n_free_g((size_t)G, 0), n_seg_g((size_t)G, 0);
  for (int64_t rid : p->trunc_order) {
    Request* r = find_req(p, rid);
    for (int g = 0; g < G; ++g) {
      const auto& st = r->step[g];
      if (st.removals.empty()) continue;
      RunInfo ri;
      ri.g = g;
      int64_t lo = st.removals[0].start, removed = 0;
      for (auto& rm : st.removals) {
        lo = std::min(lo, rm.start);
        removed += rm.end - rm.start;
      }
      ri.lo = lo;
      ri.n = std::max<int64_t>(st.removals.front().active - lo - removed, 0);
      if (!build_row_map(st.removals, lo, ri.map)) {
        p->last_error = "more than " + std::to_string(kRunRemovalsMax) + " span removals of one request and group "
                        "in one step";
        return ABKV_ERR_ARG;
      }
      // moved rows [t_star, n); A = moved rows whose source is a row of the run, [t_star, a_end); B = f(A); the
      // ordered ops are A u B (|B| = |A|, |A n B| = rows of A whose source lies in A)
      ri.t_star = ri.map.m ? std::min(ri.map.tau[0], ri.n) : ri.n;
      ri.n_moved = ri.n - ri.t_star;
      ri.a_end = std::max(std::min(ri.map.inv(ri.n), ri.n), ri.t_star);
      const int64_t nA = ri.a_end - ri.t_star;
      const int64_t nAB = std::max<int64_t>(std::min(ri.a_end, ri.map.inv(ri.a_end)) - ri.t_star, 0);
      ri.n_ch = 2 * nA - nAB;
      ri.blocks = &st.blocks_before;
      ri.blocks_lo = st.blocks_lo;
      ri.win_lo = p->page_of(lo);
      ri.win_n = p->page_of(std::max<int64_t>(st.removals.front().active - 1, lo)) - ri.win_lo + 1;
      if (ri.win_lo < ri.blocks_lo || ri.win_lo + ri.win_n > ri.blocks_lo + (int64_t)st.blocks_before.size()) {
        p->last_error = "a run's rows lie past its page list";
        return ABKV_ERR_ARG;
      }
      n_ord_g[(size_t)g] += ri.n_ch;
      n_free_g[(size_t)g] += ri.n_moved - ri.n_ch;
      n_seg_g[(size_t)g] += ri.n_ch > 0;
      infos.push_back(ri);
    }
  }
  // the layout of abkv_planner_take_moves_packed
  std::vector<int64_t> ops_at((size_t)G), offs_at((size_t)G), ord_cur((size_t)G, 0), free_cur((size_t)G, 0),
      seg_cur((size_t)G, 0);
  int64_t at = 0;
  for (int g = 0; g < G; ++g) {
    const int64_t n_ord = n_ord_g[(size_t)g], n_free = n_free_g[(size_t)g], n_seg = n_seg_g[(size_t)g];
    const int64_t pad = (n_seg + 1 + 3) & ~(int64_t)3;
    ops_at[(size_t)g] = at;
    offs_at[(size_t)g] = at + 4 * (n_ord + n_free);
    int64_t* ix = index + 5 * g;
    ix[0] = at;
    ix[1] = n_ord + n_free;
    ix[2] = offs_at[(size_t)g];
    ix[3] = n_seg;
    ix[4] = n_free;
    groups[4 * g + 0] = (int32_t)offs_at[(size_t)g];
    groups[4 * g + 1] = (int32_t)n_seg;
    groups[4 * g + 2] = (int32_t)(offs_at[(size_t)g] + pad);
    groups[4 * g + 3] = 0;
    at += 4 * (n_ord + n_free) + pad;
  }
  if (at > INT32_MAX) {
    p->last_error = "move lists exceed 2^31 int32 elements";
    return ABKV_ERR_ARG;
  }
  int64_t nr = 0, np = 0;
  for (const RunInfo& ri : infos) {
    const size_t g = (size_t)ri.g;
    const int64_t ord_base = ord_cur[g], free_base = free_cur[g];
    ord_cur[g] += ri.n_ch;
    free_cur[g] += ri.n_moved - ri.n_ch;
    int64_t seg_at = -1;
    if (ri.n_ch > 0) seg_at = offs_at[g] + 1 + seg_cur[g]++;
    if (ri.n_moved == 0) continue;
    int32_t* rec = runs + kRunFields * nr++;
    rec[0] = (int32_t)ri.n;
    rec[1] = (int32_t)(ri.lo - ri.win_lo * p->block_size);
    rec[2] = (int32_t)np;
    rec[3] = (int32_t)(ops_at[g] + 4 * ord_base);
    rec[4] = (int32_t)(ops_at[g] + 4 * (n_ord_g[g] + free_base));
    rec[5] = (int32_t)ri.n_ch;
    rec[6] = (int32_t)(ri.n_moved - ri.n_ch);
    rec[7] = (int32_t)seg_at;
    rec[8] = (int32_t)ord_cur[g];
    rec[9] = ri.map.m;
    rec[10] = (int32_t)ri.t_star;
    rec[11] = (int32_t)ri.a_end;
    rec[12] = (int32_t)ri.win_n;
    rec[13] = 0;
    for (int j = 0; j < kRunRemovalsMax; ++j) {
      rec[14 + j] = j < ri.map.m ? (int32_t)ri.map.tau[j] : 0;
      rec[14 + kRunRemovalsMax + j] = j < ri.map.m ? (int32_t)ri.map.c[j] : 0;
    }
    for (int64_t k = 0; k < ri.win_n; ++k) pages[np++] = (*ri.blocks)[(size_t)(ri.win_lo - ri.blocks_lo + k)];
  }
  int64_t t = 0;
  if (trunc_rows) {
    for (int64_t rid : p->trunc_order) {
      Request* r = find_req(p, rid);
      int64_t* row = trunc_rows + (1 + G) * t++;
      row[0] = rid;
      for (int g = 0; g < G; ++g) row[1 + g] = r->trunc[g];
    }
  }
  if (n_trunc) *n_trunc = trunc_rows ? t : need_trunc;
  sizes[0] = nr;
  sizes[1] = np;
  sizes[2] = at;
  for (auto& kv : p->reqs) {
    for (auto& st : kv.second.step) st.reset();
    kv.second.has_trunc = false;
    kv.second.alloc_after_removal = false;
  }
  p->pending_order.clear();
  p->trunc_order.clear();
  return ABKV_OK;
}

// Device-ready move lists of a step's fused rows (the fused_rows of abkv_planner_take_step_outputs; the rows of one
// (request, group) contiguous and in emission order). Within a (request, group) run, op j *depends on* op i when
// op j's destination is op i's source (j must store after i loads). Ops on such an edge are kept in one ordered
// segment per run, in emission order (the walker's order matters there); every other op reads a slot no op writes
// and writes a slot no op reads, so it is independent. Per group g < num_groups, in `out` back to back: the ops
// [n_g, 4] int32 (src_block, src_off, dst_block, dst_off) -- the ordered segments first, then the independent ops --
// followed by the segment offsets [n_segments + 1] relative to the group's first op (the last one is where the
// independent ops start). index [num_groups, 5] = (ops_at, n_ops, offs_at, n_segments, n_free), positions in int32
// elements of `out`; each group's section starts at a multiple of 4 elements (16 bytes). Returns the elements
// written; ABKV_ERR_CAPACITY if out_cap < 5 * n + 4 * num_groups; ABKV_ERR_ARG for a group outside
// [0, num_groups), a (request, group) run that appears twice, an offset outside [0, 65536), a slot read by two ops,
// or an op that reads a slot an earlier op of its run writes.
int64_t abkv_moves_pack(const int64_t* fused_rows, int64_t n, int num_groups, int32_t* out, int64_t out_cap,
                        int64_t* index) {
  if (n < 0 || num_groups <= 0 || (n > 0 && !fused_rows) || !out || !index) return ABKV_ERR_ARG;
  if (out_cap < 5 * n + 4 * (int64_t)num_groups) return ABKV_ERR_CAPACITY;
  const int G = num_groups;
  struct Run {
    int64_t lo, hi, n_chained;
  };
  std::vector<std::vector<Run>> runs((size_t)G);
  std::vector<int64_t> n_ops((size_t)G, 0), n_chained((size_t)G, 0);
  std::vector<uint8_t> chained((size_t)n, 0);
  std::unordered_map<int64_t, int> seen;                 // (request, group) -> 1
  std::vector<int64_t> tkey;
  std::vector<int32_t> tidx;
  auto slot_key = [](int64_t block, int64_t off) { return (block << 16) | off; };
  auto slot_hash = [](int64_t k, size_t cap) {
    return (size_t)((uint64_t)k * 0x9E3779B97F4A7C15ull >> 20) & (cap - 1);
  };
  for (int64_t lo = 0; lo < n;) {
    const int64_t rid = fused_rows[6 * lo], g = fused_rows[6 * lo + 1];
    if (g < 0 || g >= G) return ABKV_ERR_ARG;
    int64_t hi = lo + 1;
    while (hi < n && fused_rows[6 * hi] == rid && fused_rows[6 * hi + 1] == g) ++hi;
    if (!seen.emplace(rid * G + g, 1).second) return ABKV_ERR_ARG;
    // open-addressing table of the run's source slots -> op index
    const int64_t m = hi - lo;
    size_t cap = 16;
    while ((int64_t)cap < 2 * m) cap <<= 1;
    tkey.assign(cap, -1);
    tidx.assign(cap, -1);
    for (int64_t i = lo; i < hi; ++i) {
      const int64_t* r = fused_rows + 6 * i;
      if (r[3] < 0 || r[3] >= 65536 || r[5] < 0 || r[5] >= 65536 || r[2] < 0 || r[4] < 0) return ABKV_ERR_ARG;
      const int64_t k = slot_key(r[2], r[3]);
      size_t h = slot_hash(k, cap);
      while (tkey[h] != -1) {
        if (tkey[h] == k) return ABKV_ERR_ARG;           // one slot read by two ops
        h = (h + 1) & (cap - 1);
      }
      tkey[h] = k;
      tidx[h] = (int32_t)(i - lo);
    }
    int64_t nc = 0;
    for (int64_t j = lo; j < hi; ++j) {
      const int64_t* r = fused_rows + 6 * j;
      const int64_t k = slot_key(r[4], r[5]);
      size_t h = slot_hash(k, cap);
      while (tkey[h] != -1 && tkey[h] != k) h = (h + 1) & (cap - 1);
      if (tkey[h] == k) {
        const int64_t i = lo + tidx[h];
        if (i > j) return ABKV_ERR_ARG;                  // a later op would read what this one wrote
        nc += !chained[(size_t)i];
        chained[(size_t)i] = 1;
        nc += !chained[(size_t)j];
        chained[(size_t)j] = 1;
      }
    }
    runs[(size_t)g].push_back({lo, hi, nc});
    n_ops[(size_t)g] += m;
    n_chained[(size_t)g] += nc;
    lo = hi;
  }
  int64_t at = 0;
  for (int g = 0; g < G; ++g) {
    int32_t* ops = out + at;
    int32_t* offs = ops + 4 * n_ops[(size_t)g];
    int64_t k_ord = 0, k_free = n_chained[(size_t)g], n_seg = 0;
    offs[0] = 0;
    for (const Run& r : runs[(size_t)g]) {
      for (int64_t i = r.lo; i < r.hi; ++i) {
        const int64_t* f = fused_rows + 6 * i;
        int32_t* d = ops + 4 * (chained[(size_t)i] ? k_ord++ : k_free++);
        d[0] = (int32_t)f[2];
        d[1] = (int32_t)f[3];
        d[2] = (int32_t)f[4];
        d[3] = (int32_t)f[5];
      }
      if (r.n_chained) offs[++n_seg] = (int32_t)k_ord;
    }
    for (int64_t k2 = n_seg + 1; k2 < ((n_seg + 1 + 3) & ~(int64_t)3); ++k2) offs[k2] = 0;   // alignment padding
    int64_t* ix = index + 5 * g;
    ix[0] = at;
    ix[1] = n_ops[(size_t)g];
    ix[2] = at + 4 * n_ops[(size_t)g];
    ix[3] = n_seg;
    ix[4] = n_ops[(size_t)g] - n_chained[(size_t)g];
    at += 4 * n_ops[(size_t)g] + ((n_seg + 1 + 3) & ~(int64_t)3);
  }
  return at;
}

int64_t abkv_planner_num_free(void* h) {
  Planner* p = static_cast<Planner*>(h);
  return p ? (int64_t)p->free_q.size() : -1;
}

int64_t abkv_planner_free_queue(void* h, int32_t* out, int64_t cap) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  if ((int64_t)p->free_q.size() > cap) return ABKV_ERR_CAPACITY;
  int64_t i = 0;
  for (int32_t b : p->free_q) out[i++] = b;
  return i;
}

int64_t abkv_planner_block_ids(void* h, int64_t rid, int group, int32_t* out, int64_t cap) {
  Planner* p = static_cast<Planner*>(h);
  if (!p || group < 0 || group >= p->num_groups) return ABKV_ERR_ARG;
  Request* r = find_req(p, rid);
  if (!r) return ABKV_ERR_NO_REQUEST;
  auto& bl = r->blocks[group];
  if ((int64_t)bl.size() > cap) return ABKV_ERR_CAPACITY;
  for (size_t i = 0; i < bl.size(); ++i) out[i] = bl[i];
  return (int64_t)bl.size();
}

// Write the page lists of `n` requests for one group into a [n, stride] int32 table (unused entries = pad).
int abkv_planner_fill_block_table(void* h, const int64_t* rids, int n, int group, int32_t* table, int64_t stride,
                                  int32_t pad) {
  Planner* p = static_cast<Planner*>(h);
  if (!p || group < 0 || group >= p->num_groups) return ABKV_ERR_ARG;
  for (int i = 0; i < n; ++i) {
    Request* r = find_req(p, rids[i]);
    if (!r) return ABKV_ERR_NO_REQUEST;
    auto& bl = r->blocks[group];
    if ((int64_t)bl.size() > stride) return ABKV_ERR_CAPACITY;
    int32_t* row = table + (int64_t)i * stride;
    for (int64_t k = 0; k < stride; ++k) row[k] = k < (int64_t)bl.size() ? bl[k] : pad;
  }
  return ABKV_OK;
}

int64_t abkv_planner_compacted(void* h, int64_t rid, int group) {
  Planner* p = static_cast<Planner*>(h);
  if (!p || group < 0 || group >= p->num_groups) return ABKV_ERR_ARG;
  Request* r = find_req(p, rid);
  return r ? r->spans[group].total : ABKV_ERR_NO_REQUEST;
}

int64_t abkv_planner_spans(void* h, int64_t rid, int group, int64_t* out, int64_t cap) {
  Planner* p = static_cast<Planner*>(h);
  if (!p || group < 0 || group >= p->num_groups) return ABKV_ERR_ARG;
  Request* r = find_req(p, rid);
  if (!r) return ABKV_ERR_NO_REQUEST;
  auto& sp = r->spans[group].spans;
  if ((int64_t)sp.size() > cap) return ABKV_ERR_CAPACITY;
  for (size_t i = 0; i < sp.size(); ++i) {
    out[2 * i] = sp[i].first;
    out[2 * i + 1] = sp[i].second;
  }
  return (int64_t)sp.size();
}

int64_t abkv_planner_logical_to_physical(void* h, int64_t rid, int group, int64_t pos) {
  Planner* p = static_cast<Planner*>(h);
  if (!p || group < 0 || group >= p->num_groups) return ABKV_ERR_ARG;
  Request* r = find_req(p, rid);
  return r ? r->spans[group].l2p(pos) : ABKV_ERR_NO_REQUEST;
}

int64_t abkv_planner_physical_to_logical(void* h, int64_t rid, int group, int64_t pos) {
  Planner* p = static_cast<Planner*>(h);
  if (!p || group < 0 || group >= p->num_groups) return ABKV_ERR_ARG;
  Request* r = find_req(p, rid);
  return r ? r->spans[group].p2l(pos) : ABKV_ERR_NO_REQUEST;
}

int abkv_planner_is_token_active(void* h, int64_t rid, int group, int64_t pos) {
  Planner* p = static_cast<Planner*>(h);
  if (!p || group < 0 || group >= p->num_groups) return ABKV_ERR_ARG;
  Request* r = find_req(p, rid);
  return r ? (r->spans[group].is_active(pos) ? 1 : 0) : ABKV_ERR_NO_REQUEST;
}

// Apply a batch of scheduler events. Each event is 6 int64: (kind, rid, a, b, group_mask, 0) with
//   kind 0: add request rid
//   kind 1: schedule a tokens: allocate_slots(rid, a) then num_computed += a (must succeed)
//   kind 2: mask_token_span(rid, a, b, groups = bits of group_mask, or all groups when group_mask < 0)
//   kind 3: free request rid
//   kind 4: take (and drop) the step outputs
// Returns the number of events applied; on failure stops and returns -(index + 1) with last_error set.
int64_t abkv_planner_apply_events(void* h, const int64_t* ev, int64_t n) {
  Planner* p = static_cast<Planner*>(h);
  if (!p) return ABKV_ERR_ARG;
  std::vector<int32_t> gl;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t* e = ev + 6 * i;
    int rc = ABKV_OK;
    switch (e[0]) {
      case 0:
        rc = abkv_planner_add_request(h, e[1]);
        break;
      case 1: {
        rc = abkv_planner_allocate_slots(h, e[1], e[2]);
        if (rc == 0) {
          p->last_error = "pool exhausted";
          rc = ABKV_ERR_POOL;
        } else if (rc == 1) {
          rc = ABKV_OK;
          find_req(p, e[1])->num_computed += e[2];
        }
        break;
      }
      case 2: {
        gl.clear();
        if (e[4] >= 0)
          for (int g = 0; g < p->num_groups; ++g)
            if ((e[4] >> g) & 1) gl.push_back(g);
        rc = abkv_planner_mask_token_span(h, e[1], e[2], e[3], e[4] >= 0 ? gl.data() : nullptr,
                                          e[4] >= 0 ? (int)gl.size() : -1, nullptr, nullptr);
        break;
      }
      case 3:
        rc = abkv_planner_free_request(h, e[1]);
        break;
      case 4:
        rc = abkv_planner_take_step_outputs(h, nullptr, 0, nullptr, nullptr, 0, nullptr, nullptr, 0, nullptr);
        break;
      default:
        p->last_error = "unknown event kind";
        rc = ABKV_ERR_ARG;
    }
    if (rc != ABKV_OK) return -(i + 1);
  }
  return n;
}

}  // extern "C"
