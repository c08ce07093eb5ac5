// Host-side planning of one encoder forward (plain C++, no device code):
// the micro-batch groups and the attention work items. The encoder
// (model.cpp) uploads the result; tests/cpp/test_plan.cpp checks it on the
// CPU.
#pragma once

#include <cstdint>
#include <vector>

namespace fa {

constexpr int kMaxMicrobatches = 4;  // streams a forward may use (micro-batches)
constexpr int kXcds = 8;             // MI355X: a launch's workgroup i runs on XCD i % 8

// Cuts B sequences (M tokens in all) into min(want, B) contiguous groups of
// about equal token count, each holding at least one sequence: group g is
// sequences [gb[g], gb[g+1]). Returns the number of groups (1 when want <=
// 1). gb holds kMaxMicrobatches + 1 entries; want <= kMaxMicrobatches.
int plan_groups(const int32_t* lengths, int B, int64_t M, int want, int* gb);

struct AttnPlanIn {
  const int32_t* lengths = nullptr;  // B lengths, each 1..T
  int B = 0, T = 0, H = 0;           // H query heads (every layer)
  const int* layer_D = nullptr;      // head dim of each of the model's layers
  const int* layer_Hkv = nullptr;    // key/value heads of each layer
  int n_layers = 0;
  int n_run = 0;                     // layers this forward runs (the first n_run)
  int groups = 1;
  const int* gb = nullptr;           // [groups + 1] from plan_groups
  int cus = 256;
  // kernel geometry: keys per tile of the tile attention, queries per fp32
  // item, the most key runs per item, and the largest batch (tokens) that
  // the fp32 attention cuts into key runs
  int tile_keys = 32, varlen_qblock = 32, max_key_parts = 8;
  int64_t split_rows = 1024;
  int forced_key_parts = 0;          // tuning: key runs forced (0: chosen)
  int forced_rows = 0;               // tuning: tile item rows forced, 64 or 128 (0: chosen)
  int forced_xcd = 0;                // tuning: XCD-local item order forced on (1) or off (-1)
  int64_t tile_min_rows = 1024;      // the tile attention from more tokens than this,
  int64_t tile_min_pairs = 458752;   // or from this many query-key pairs per head (sum L^2)
};

struct AttnPlan {
  int64_t M = 0;                      // tokens
  bool tiles_ok = false;              // the batch may take the tile attention
  bool mixed_hkv = false;             // the head_dim-256 layers differ in kv heads
  bool any_tiles = false, any_var = false;  // some run layer takes each path
  int hkv_t = 0;                      // kv heads of the tile layers
  int Gt = 1;                         // query heads per kv head of the tile layers
  int waves_t = 8;                    // 16-row blocks per tile item: 8 (128 rows) or 4 (64 rows)
  int kparts_t = 1, kparts_v = 1;     // key runs per tile item, per fp32 item
  int64_t n_items_t = 0, n_items_v = 0;
  int64_t n_tiles = 0;                // key tiles over the batch (tile layers)
  int64_t group_items_t[kMaxMicrobatches] = {}, group_items_v[kMaxMicrobatches] = {};
  // whether each group's items took the XCD-local order (plan_items)
  bool xcd_local_t[kMaxMicrobatches] = {}, xcd_local_v[kMaxMicrobatches] = {};
  // does a layer of head_dim D take the tile attention?
  bool layer_tiles(int D) const { return tiles_ok && !mixed_hkv && D == 256; }
};

// Chooses each layer's attention path, the tile items' wave count and the
// key runs of both kinds of item, and counts items and key tiles.
void plan_attention(const AttnPlanIn& in, AttnPlan& p);

// Writes the items, 3 ints each: first the tile items (sequence, first row,
// kv head), then the fp32 items (sequence, first query, head), each list
// ordered by group and, within a group, longest sequences first; items of
// one workgroup each (kparts == 1) instead go to per-XCD queues, a
// sequence's items together where the queues' balance allows (longest first
// within a queue), interleaved by position, where that order's estimated
// span is within 3 % of the plain order's (p.xcd_local_t / _v); fills
// p.group_items_t and p.group_items_v. items holds 3 * (p.n_items_t +
// p.n_items_v) ints; order is scratch.
void plan_items(const AttnPlanIn& in, AttnPlan& p, int32_t* items, std::vector<int>& order);

}  // namespace fa
