// The encoder's host-side plan (ai_amd/csrc/plan.cpp) on the CPU: micro-batch
// groups and attention work items for EmbeddingGemma-300M and EmbeddingGemma
// 2 layer stacks at the configs' shapes. Checks what the kernels rely on:
// every (row, kv head) or (query, head) of every sequence in exactly one
// item, items of a group from that group's sequences only, groups
// contiguous and token-balanced, and the path, wave-count and key-run
// choices at their thresholds. Run by tests/test_cpp_host.py.
#include <algorithm>
#include <map>
#include <set>
#include <numeric>
#include <tuple>
#include <vector>

#include "plan.h"
#include "testing.hpp"

using fa::AttnPlan;
using fa::AttnPlanIn;

namespace {

struct Stack {
  std::vector<int> D, Hkv;
  int H;
};

Stack eg300m() { return {std::vector<int>(24, 256), std::vector<int>(24, 1), 3}; }

// EmbeddingGemma 2 (TestConfig2): 12 layers, full attention on 5 and 11
// with head_dim 512 and one kv head, sliding layers head_dim 256, 2 kv heads
Stack eg2() {
  Stack s{std::vector<int>(12, 256), std::vector<int>(12, 2), 4};
  for (int l : {5, 11}) {
    s.D[l] = 512;
    s.Hkv[l] = 1;
  }
  return s;
}

struct Case {
  std::vector<int32_t> lengths;
  int T = 0;
  int groups = 1;
  int gb[fa::kMaxMicrobatches + 1] = {};
  AttnPlanIn in;
  AttnPlan p;
  std::vector<int32_t> items;
};

void run(Case& c, const Stack& s, int want_groups, int n_run = -1) {
  const int B = (int)c.lengths.size();
  c.T = *std::max_element(c.lengths.begin(), c.lengths.end());
  const int64_t M = std::accumulate(c.lengths.begin(), c.lengths.end(), int64_t{0});
  c.gb[0] = 0;
  c.gb[1] = B;
  c.groups = want_groups > 1 ? fa::plan_groups(c.lengths.data(), B, M, want_groups, c.gb) : 1;
  c.in.lengths = c.lengths.data();
  c.in.B = B;
  c.in.T = c.T;
  c.in.H = s.H;
  c.in.layer_D = s.D.data();
  c.in.layer_Hkv = s.Hkv.data();
  c.in.n_layers = (int)s.D.size();
  c.in.n_run = n_run < 0 ? (int)s.D.size() : n_run;
  c.in.groups = c.groups;
  c.in.gb = c.gb;
  fa::plan_attention(c.in, c.p);
  c.items.assign(3 * (c.p.n_items_t + c.p.n_items_v), -1);
  std::vector<int> order;
  fa::plan_items(c.in, c.p, c.items.data(), order);
}

// Every row block of every sequence (and head) in exactly one item of its
// group's run; groups in order; within a group, longest sequences first —
// for items of one workgroup each, within each XCD's positions (i % 8),
// and sequences spread over more than one XCD only where a queue filled
// up, which each of the 8 queues does once: at most 8 extra XCDs over the
// group's sequences.
void check_items(const Case& c) {
  const AttnPlan& p = c.p;
  int64_t it = 0;
  for (int list = 0; list < 2; list++) {
    const bool tiles = list == 0;
    if (!(tiles ? p.any_tiles : p.any_var)) {
      for (int g = 0; g < c.groups; g++)
        if ((tiles ? p.group_items_t : p.group_items_v)[g] != 0) FATAL("unused list %d has items", list);
      continue;
    }
    const int istep = tiles ? 16 * p.waves_t : c.in.varlen_qblock;
    const int iheads = tiles ? p.hkv_t : c.in.H;
    std::map<std::tuple<int, int, int>, int> seen;
    for (int g = 0; g < c.groups; g++) {
      const bool xcd = (tiles ? p.kparts_t == 1 : p.kparts_v == 1) && (tiles ? p.xcd_local_t : p.xcd_local_v)[g];
      const int64_t n = (tiles ? p.group_items_t : p.group_items_v)[g];
      int prev_len = 1 << 30;
      if (xcd) {
        int prev_x[fa::kXcds];
        for (int& v : prev_x) v = 1 << 30;
        std::map<int, std::set<int>> residues;
        for (int64_t k = 0; k < n; k++) {
          const int b = c.items[3 * (it + k)], x = (int)(k % fa::kXcds);
          residues[b].insert(x);
          if (c.lengths[b] > prev_x[x]) FATAL("group %d, XCD %d: sequence %d (length %d) after a shorter one", g, x, b, c.lengths[b]);
          prev_x[x] = c.lengths[b];
        }
        // a sequence moves to another queue only when its queue is full
        int64_t spills = 0;
        for (auto& [b, r] : residues) spills += (int64_t)r.size() - 1;
        if (spills > fa::kXcds)
          FATAL("group %d: sequences spread over %lld extra XCDs", g, (long long)spills);
      }
      for (int64_t k = 0; k < n; k++, it++) {
        const int b = c.items[3 * it], q0 = c.items[3 * it + 1], h = c.items[3 * it + 2];
        if (b < c.gb[g] || b >= c.gb[g + 1]) FATAL("item %lld of group %d: sequence %d outside [%d, %d)", (long long)it, g, b, c.gb[g], c.gb[g + 1]);
        const int rows = tiles ? p.Gt * c.lengths[b] : c.lengths[b];
        if (q0 < 0 || q0 >= rows || q0 % istep != 0) FATAL("item %lld: first row %d of %d (step %d)", (long long)it, q0, rows, istep);
        if (h < 0 || h >= iheads) FATAL("item %lld: head %d of %d", (long long)it, h, iheads);
        if (!xcd && c.lengths[b] > prev_len) FATAL("group %d: sequence %d (length %d) after a shorter one", g, b, c.lengths[b]);
        prev_len = c.lengths[b];
        if (seen[{b, q0, h}]++) FATAL("item (%d, %d, %d) twice", b, q0, h);
      }
    }
    int64_t want = 0;
    for (size_t b = 0; b < c.lengths.size(); b++) {
      const int rows = tiles ? p.Gt * c.lengths[b] : c.lengths[b];
      want += (int64_t)((rows + istep - 1) / istep) * iheads;
    }
    if ((int64_t)seen.size() != want) FATAL("list %d: %zu distinct items, want %lld", list, seen.size(), (long long)want);
    if (want != (tiles ? p.n_items_t : p.n_items_v)) FATAL("list %d: counted %lld items, wrote %lld", list, (long long)(tiles ? p.n_items_t : p.n_items_v), (long long)want);
  }
  if (it != p.n_items_t + p.n_items_v) FATAL("wrote %lld items of %lld", (long long)it, (long long)(p.n_items_t + p.n_items_v));
}

std::vector<int32_t> repeat(int n, int len) { return std::vector<int32_t>(n, len); }

}  // namespace

// plan_groups: contiguous, non-empty, every sequence once, and each group's
// tokens within one sequence of its share
TEST(TestGroupsBalanced) {
  std::vector<int32_t> lengths;
  uint32_t x = 12345;
  for (int b = 0; b < 37; b++) {
    x = x * 1664525u + 1013904223u;
    lengths.push_back(20 + (int)(x >> 24));  // 20..275
  }
  const int B = (int)lengths.size();
  const int64_t M = std::accumulate(lengths.begin(), lengths.end(), int64_t{0});
  const int maxlen = *std::max_element(lengths.begin(), lengths.end());
  for (int want = 1; want <= fa::kMaxMicrobatches; want++) {
    int gb[fa::kMaxMicrobatches + 1];
    const int g = fa::plan_groups(lengths.data(), B, M, want, gb);
    if (g != want) FATAL("want %d groups, got %d", want, g);
    if (gb[0] != 0 || gb[g] != B) FATAL("groups cover [%d, %d)", gb[0], gb[g]);
    for (int i = 0; i < g; i++) {
      if (gb[i + 1] <= gb[i]) FATAL("group %d empty", i);
      int64_t tok = 0;
      for (int b = gb[i]; b < gb[i + 1]; b++) tok += lengths[b];
      if (std::abs((double)tok - (double)M / g) > maxlen) FATAL("group %d of %d: %lld tokens of %lld", i, g, (long long)tok, (long long)M);
    }
  }
  // more groups than sequences: one sequence each
  int gb[fa::kMaxMicrobatches + 1];
  const int32_t two[] = {5, 900};
  if (fa::plan_groups(two, 2, 905, 3, gb) != 2 || gb[1] != 1 || gb[2] != 2) FATAL("two sequences, three groups wanted");
}

// C1 (one 128-token sentence): the fp32 kernel, 12 items cut into 8 key
// runs of one 16-key tile
TEST(TestC1FP32KeyRuns) {
  Case c;
  c.lengths = {128};
  run(c, eg300m(), 1);
  if (c.p.any_tiles || !c.p.any_var) FATAL("C1 takes the fp32 kernel");
  if (c.p.n_items_v != 12 || c.p.kparts_v != 8) FATAL("items %lld key runs %d, want 12 and 8", (long long)c.p.n_items_v, c.p.kparts_v);
  check_items(c);
}

// The fp32 items' key runs: at most one per 16-key tile and per CU share,
// no more than the run length needs, none from two tiles down
TEST(TestFP32KeyRunCounts) {
  struct K { std::vector<int32_t> lengths; int items, runs; };
  const K cases[] = {
      {{32}, 3, 1},                 // two tiles: no runs (no combine launch)
      {{48}, 6, 3},                 // three tiles of one key run each
      {{64}, 6, 4},
      {{300}, 30, 7},               // 8 CU shares of 19 tiles: runs of 3 tiles, 7 of them
      {{500}, 48, 5},               // 5 CU shares of 32 tiles: runs of 7 tiles
      {{128, 128, 128, 128}, 48, 4}, // 5 CU shares of 8 tiles: runs of 2, 4 of them
  };
  for (const K& k : cases) {
    Case c;
    c.lengths = k.lengths;
    run(c, eg300m(), 1);
    if (c.p.any_tiles || !c.p.any_var) FATAL("%d tokens: the fp32 kernel expected", (int)k.lengths[0]);
    if (c.p.n_items_v != k.items || c.p.kparts_v != k.runs)
      FATAL("%zu x %d: items %lld key runs %d, want %d and %d", k.lengths.size(), (int)k.lengths[0],
            (long long)c.p.n_items_v, c.p.kparts_v, k.items, k.runs);
    check_items(c);
  }
}

// over 1 024 tokens at >= 32 per sequence: the tile attention; the wave
// count by the 128-row item count against 256 CUs
TEST(TestTileWaves) {
  const struct {
    int n, len, waves;
    int64_t items;  // items of the chosen wave count
  } cases[] = {
      {43, 128, 4, 43 * 6},   // 129 items of 128 rows: just over half a round
      {52, 128, 8, 52 * 3},   // 156: just over 0.6 of a round
      {36, 160, 4, 36 * 8},   // 144 items of 128 rows: 0.56 of a round
      {40, 160, 8, 40 * 4},   // 160: 0.63
      {48, 160, 8, 48 * 4},   // 192
      {8, 2048, 8, 8 * 48},   // C4-like, one round and a half
  };
  for (const auto& tc : cases) {
    Case c;
    c.lengths = repeat(tc.n, tc.len);
    run(c, eg300m(), 3);
    if (!c.p.any_tiles || c.p.any_var) FATAL("%d x %d: tile attention on every layer", tc.n, tc.len);
    if (c.p.waves_t != tc.waves) FATAL("%d x %d: %d waves, want %d", tc.n, tc.len, c.p.waves_t, tc.waves);
    if (c.p.n_items_t != tc.items) FATAL("%d x %d: %lld items, want %lld", tc.n, tc.len, (long long)c.p.n_items_t, (long long)tc.items);
    if (c.p.kparts_t != 1) FATAL("%d x %d: %d key runs", tc.n, tc.len, c.p.kparts_t);
    if (c.p.n_tiles != (int64_t)tc.n * ((tc.len + 31) / 32)) FATAL("key tiles %lld", (long long)c.p.n_tiles);
    check_items(c);
  }
  // the same batch on one stream (no micro-batches): eight waves (equal
  // lengths: the pairs' second round would only add time)
  Case c;
  c.lengths = repeat(36, 160);
  run(c, eg300m(), 1);
  if (c.p.waves_t != 8 || c.p.n_items_t != 36 * 4) FATAL("one stream: %d waves, %lld items", c.p.waves_t, (long long)c.p.n_items_t);
  check_items(c);
  // a ragged batch at the same fill on one stream (longest 1.25x the mean
  // or more): pairs. 20 x 100 + 14 x 220 tokens: 20 x 3 + 14 x 6 = 144
  // items of 128 rows (0.56 of a round), mean 149, longest 220
  Case r;
  r.lengths = repeat(20, 100);
  for (int i = 0; i < 14; i++) r.lengths.push_back(220);
  run(r, eg300m(), 1);
  if (r.p.waves_t != 4 || r.p.n_items_t != 20 * 5 + 14 * 11)
    FATAL("ragged one stream: %d waves, %lld items", r.p.waves_t, (long long)r.p.n_items_t);
  check_items(r);
}

// one stream, at most half a round of 128-row items, sequences under 1 536
// tokens: 64-row items (waves_t 4), key runs by the doubled item count
TEST(TestOneStreamFewItems) {
  Case c;
  c.lengths = {1100};  // 26 items of 128 rows -> 52 of 64
  run(c, eg300m(), 1);
  if (c.p.waves_t != 4 || c.p.n_items_t != 52 || c.p.kparts_t != 4)
    FATAL("waves %d items %lld key runs %d, want 4, 52, 4", c.p.waves_t, (long long)c.p.n_items_t, c.p.kparts_t);
  check_items(c);
  Case d;
  d.lengths = repeat(8, 160);  // 32 items of 128 rows
  run(d, eg300m(), 1);
  if (d.p.waves_t != 4 || d.p.n_items_t != 64) FATAL("8 x 160: waves %d items %lld", d.p.waves_t, (long long)d.p.n_items_t);
  check_items(d);
}

// one long sequence: 48 items of 128 rows, keys cut into 5 runs of 12-13 tiles
TEST(TestTileKeyRuns) {
  Case c;
  c.lengths = {2048};
  run(c, eg300m(), 1);
  if (c.p.waves_t != 8 || c.p.n_items_t != 48 || c.p.kparts_t != 5)
    FATAL("waves %d items %lld key runs %d, want 8, 48, 5", c.p.waves_t, (long long)c.p.n_items_t, c.p.kparts_t);
  check_items(c);
}

// short sequences (under 32 tokens on average) keep the fp32 kernel
TEST(TestShortSequencesFP32) {
  Case c;
  c.lengths = repeat(64, 20);  // 1 280 tokens
  run(c, eg300m(), 1);
  if (c.p.tiles_ok || c.p.any_tiles) FATAL("20-token sequences take the tile attention");
  check_items(c);
}

// the tile attention's batch rules at their edges: more than 1 024 tokens
// or at least 458 752 query-key pairs per head, and at least 32 tokens per
// sequence on average
TEST(TestTilePathBoundaries) {
  struct Edge {
    std::vector<int32_t> lengths;
    bool tiles;
  };
  std::vector<int32_t> l1025 = repeat(7, 128), l1055 = repeat(32, 32);
  l1025.push_back(129);
  l1055.push_back(31);
  const Edge edges[] = {{repeat(8, 128), false}, {l1025, true}, {l1055, false}, {repeat(33, 32), true},
                        {{512, 512}, true},    // 524 288 pairs
                        {{384, 384}, false},   // 294 912
                        {{640}, false},        // 409 600
                        {{678}, true},         // 459 684
                        {{677}, false}};       // 458 329
  for (const Edge& e : edges) {
    for (int want : {1, 3}) {
      Case c;
      c.lengths = e.lengths;
      run(c, eg300m(), want);
      if (c.p.tiles_ok != e.tiles || c.p.any_tiles != e.tiles || c.p.any_var == e.tiles)
        FATAL("%zu sequences, %lld tokens, %d groups: tiles %d, want %d", e.lengths.size(), (long long)c.p.M, c.groups,
              (int)c.p.any_tiles, (int)e.tiles);
      check_items(c);
    }
  }
}

// EmbeddingGemma 2: sliding layers on the tiles (2 kv heads, 2 query heads
// each), full layers (head_dim 512) on the fp32 kernel; both lists by group
TEST(TestEG2TwoLists) {
  Case c;
  c.lengths = {256, 131, 200, 77, 256, 160, 90, 199, 240, 64, 180, 222};
  run(c, eg2(), 3);
  if (!c.p.any_tiles || !c.p.any_var) FATAL("both paths expected");
  if (c.p.hkv_t != 2 || c.p.Gt != 2) FATAL("kv heads %d, query heads per kv head %d", c.p.hkv_t, c.p.Gt);
  if (!c.p.layer_tiles(256) || c.p.layer_tiles(512)) FATAL("per-layer path");
  check_items(c);
  // only the first five (sliding) layers run: no fp32 items
  Case d;
  d.lengths = c.lengths;
  run(d, eg2(), 3, 5);
  if (!d.p.any_tiles || d.p.any_var || d.p.n_items_v != 0) FATAL("five sliding layers: fp32 items %lld", (long long)d.p.n_items_v);
  check_items(d);
}

// head_dim-256 layers with different kv head counts keep the fp32 kernel
TEST(TestMixedKvHeads) {
  Stack s = eg300m();
  s.Hkv[3] = 3;
  Case c;
  c.lengths = repeat(16, 200);
  run(c, s, 2);
  if (!c.p.mixed_hkv || c.p.any_tiles || !c.p.any_var) FATAL("mixed kv heads must keep the fp32 kernel");
  check_items(c);
}

int main(int argc, char** argv) { return ctest::run_all(argc, argv); }

// The XCD-local order for long key loops where it does not lengthen the
// launch: equal lengths (C3-like, several rounds) take it; a C4-like batch
// on one stream (281 items of 1 024-2 048 tokens, more than one round)
// keeps the plain longest-first order, whose second round holds only the
// shortest sequence's items, and so does a C2-like batch (mean length 172:
// short key loops).
TEST(TestXcdLocalChoice) {
  {
    Case c;
    c.lengths = repeat(64, 512);
    run(c, eg300m(), 1);
    if (!c.p.xcd_local_t[0]) FATAL("C3-like, one stream: plain order");
    check_items(c);
  }
  {
    Case c;
    c.lengths = {2048, 1900, 1700, 1500, 1300, 1200, 1100, 1024};
    run(c, eg300m(), 1);
    if (c.p.kparts_t != 1) FATAL("C4-like: %d key runs", c.p.kparts_t);
    if (c.p.xcd_local_t[0]) FATAL("C4-like, one stream: XCD-local order");
    check_items(c);
  }
  {
    Case c;
    uint32_t x = 7;
    for (int b = 0; b < 32; b++) {
      x = x * 1664525u + 1013904223u;
      c.lengths.push_back(64 + (int)((x >> 8) % 193));  // U[64, 256]
    }
    for (int groups : {1, 3}) {
      run(c, eg300m(), groups);
      for (int g = 0; g < groups; g++)
        if (c.p.xcd_local_t[g]) FATAL("C2-like, %d groups: group %d in XCD-local order", groups, g);
      check_items(c);
    }
  }
  {
    Case c;  // C4-like in four micro-batches: two sequences per group, one round each
    c.lengths = {2048, 1900, 1700, 1500, 1300, 1200, 1100, 1024};
    run(c, eg300m(), 4);
    for (int g = 0; g < 4; g++)
      if (!c.p.xcd_local_t[g]) FATAL("C4-like, 4 groups: group %d in plain order", g);
    check_items(c);
  }
}
