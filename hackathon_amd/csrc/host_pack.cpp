// Host-side tick packing for process_batch (example_model.py:819-905):
// from the batch's per-symbol request counts, the engine's runs (sorted by
// non-increasing length, stable), each request's row in the tick, and the
// order in which the reference lists the answers. Host memory only; no HIP
// call.
#include <algorithm>
#include <cstdint>
#include <numeric>
#include <vector>

#include "common.h"

extern "C" {

// Items are the batch's symbols in dict order: item i has item_len[i]
// requests and slot item_slot[i] (-1: no slot, answered with zeros). The
// requests are numbered item by item (request k of item i is
// sum(item_len[:i]) + k). Outputs:
// - slot_ids[n_runs], run_off[n_runs + 1]: one run per slotted item with
//   requests, by non-increasing length, ties in item order;
// - req_row[n_req]: the row of each request (-1 for unslotted items);
// - resp_req[n_req]: the request answered at each response position: every
//   request of an unslotted item first, in item order
//   (example_model.py:826-839), then round by round (round k: the k-th
//   request of every slotted item longer than k, in item order;
//   example_model.py:881-899).
// Slots must be distinct. Returns 0, or -1 for bad arguments.
int hk_pack_tick(const int* item_slot, const int* item_len, int n_items, int* slot_ids,
                 int* run_off, int* req_row, int* resp_req, int* n_runs_out, int* n_rows_out) {
  HK_REQUIRE(n_items >= 0 && n_runs_out && n_rows_out, "hk_pack_tick: bad arguments");
  HK_REQUIRE(n_items == 0 || (item_slot && item_len && slot_ids && run_off),
             "hk_pack_tick: null item or run array");
  int64_t n_req = 0;
  std::vector<int> base(n_items);
  std::vector<int> runs;  // slotted items with requests
  runs.reserve(n_items);
  for (int i = 0; i < n_items; ++i) {
    HK_REQUIRE(item_len[i] >= 0 && item_slot[i] >= -1, "hk_pack_tick: item %d: len %d slot %d", i,
               item_len[i], item_slot[i]);
    base[i] = (int)n_req;
    n_req += item_len[i];
    HK_REQUIRE(n_req < (int64_t(1) << 31), "hk_pack_tick: too many requests");
    if (item_slot[i] >= 0 && item_len[i] > 0) runs.push_back(i);
  }
  HK_REQUIRE(n_req == 0 || (req_row && resp_req), "hk_pack_tick: null request array");
  {
    std::vector<int> slots;
    slots.reserve(runs.size());
    for (int i : runs) slots.push_back(item_slot[i]);
    std::sort(slots.begin(), slots.end());
    HK_REQUIRE(std::adjacent_find(slots.begin(), slots.end()) == slots.end(),
               "hk_pack_tick: a slot appears in two items");
  }
  std::stable_sort(runs.begin(), runs.end(),
                   [&](int a, int b) { return item_len[a] > item_len[b]; });
  run_off[0] = 0;
  for (size_t p = 0; p < runs.size(); ++p) {
    const int i = runs[p];
    slot_ids[p] = item_slot[i];
    run_off[p + 1] = run_off[p] + item_len[i];
    for (int k = 0; k < item_len[i]; ++k) req_row[base[i] + k] = run_off[p] + k;
  }
  int pos = 0;
  int max_len = 0;
  std::vector<int> live;  // slotted items still holding requests, item order
  live.reserve(runs.size());
  for (int i = 0; i < n_items; ++i) {
    if (item_slot[i] < 0) {
      for (int k = 0; k < item_len[i]; ++k) {
        req_row[base[i] + k] = -1;
        resp_req[pos++] = base[i] + k;
      }
    } else if (item_len[i] > 0) {
      live.push_back(i);
      max_len = std::max(max_len, item_len[i]);
    }
  }
  for (int k = 0; k < max_len; ++k) {
    size_t keep = 0;
    for (size_t j = 0; j < live.size(); ++j) {
      const int i = live[j];
      resp_req[pos++] = base[i] + k;
      if (item_len[i] > k + 1) live[keep++] = i;
    }
    live.resize(keep);
  }
  *n_runs_out = (int)runs.size();
  *n_rows_out = runs.empty() ? 0 : run_off[runs.size()];
  return HK_OK;
}

}  // extern "C"
