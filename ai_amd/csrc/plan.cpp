// Host-side planning of one encoder forward: micro-batch groups and
// attention work items (plan.h).
#include "plan.h"

#include <algorithm>

namespace fa {

int plan_groups(const int32_t* lengths, int B, int64_t M, int want, int* gb) {
  want = std::max(1, std::min(want, std::min(B, kMaxMicrobatches)));
  gb[0] = 0;
  int b = 0;
  int64_t cum = 0;
  for (int g = 1; g < want; g++) {
    // cut before the sequence that would take the groups so far past g/want
    // of the tokens, keeping at least one sequence in this group and in
    // each later one
    while (b < B - (want - g) && (cum + lengths[b]) * want <= M * g) cum += lengths[b++];
    if (b == gb[g - 1]) cum += lengths[b++];
    gb[g] = b;
  }
  gb[want] = B;
  return want;
}

void plan_attention(const AttnPlanIn& in, AttnPlan& p) {
  p = AttnPlan{};
  for (int b = 0; b < in.B; b++) p.M += in.lengths[b];
  // Layers with head_dim 256 (every EmbeddingGemma layer, EmbeddingGemma
  // 2's sliding layers) take the split-bf16 tile attention, from 1 025
  // tokens, or from 448·1 024 query-key pairs per head (sum of L^2) in a
  // smaller batch, with at least 32 tokens per sequence on average
  // (batches of shorter sequences keep the fp32 kernel's 16-key tiles: a
  // 32-key tile would be mostly padding). Below 1 025 tokens the pairs
  // decide (MI355X, per forward, tile vs fp32 kernel): 2 x 512 tokens
  // 2.30 vs 2.56 ms, 768 + 200 2.33 vs 2.65, one 768-token sequence 2.18
  // vs 2.30, one 1 000-token sequence 2.37 vs 2.73; but 640 tokens 2.08 vs
  // 2.06, 2 x 384 2.13 vs 2.08, 5 x 200 2.30 vs 2.14, 4 x 128 1.87 vs 1.67.
  // The tile layers share one kv head count (the item rows and image slots
  // depend on it); a model whose head_dim-256 layers differ in it keeps the
  // fp32 kernel.
  double pairs = 0;
  for (int b = 0; b < in.B; b++) pairs += (double)in.lengths[b] * in.lengths[b];
  p.tiles_ok = (p.M > in.tile_min_rows || pairs >= (double)in.tile_min_pairs) && p.M >= 32LL * in.B;
  for (int l = 0; l < in.n_layers; l++) {
    if (in.layer_D[l] != 256) continue;
    if (p.hkv_t && in.layer_Hkv[l] != p.hkv_t) p.mixed_hkv = true;
    p.hkv_t = in.layer_Hkv[l];
  }
  for (int l = 0; l < in.n_run; l++) (p.layer_tiles(in.layer_D[l]) ? p.any_tiles : p.any_var) = true;
  p.Gt = p.any_tiles ? in.H / p.hkv_t : 1;
  // Tile items of 128 rows (eight waves); of 64 rows (waves_t = 4: eight
  // waves in head-dimension pairs, or four single waves) when the batch
  // runs as micro-batches and its 128-row items would fill more than half
  // a round of the CUs but at most 0.6 of one: twice the items, each with
  // half the rows and the same key loop, still about one round, shorten
  // the attention's link in every group's chain of dependent launches (on
  // one stream the launch's own time decides: at C2 1.19 ms of attention
  // per forward with 128-row items, 1.22 with 64-row pairs). Measured per
  // forward on MI355X (256 CUs), 128- vs 64-row items (then four single
  // waves): C2 (143 items of 128 rows) 5.22 vs 5.11 ms; 36 x
  // 160 tokens (144 items) 5.09 vs 5.00; 40 x 160 (160) 5.61 vs 5.65; 48 x
  // 160 (192) 6.34 vs 6.49; EmbeddingGemma 2 at C2 (202) 4.15 vs 4.17; C3,
  // C4, C5 (from 271 items) 4-9 % slower with four. Below half a round the
  // key runs spread the work instead.
  // On one stream with at most half a round of 128-row items (the key
  // runs' regime), 64-row items on eight waves in head-dimension pairs win
  // while the sequences stay under 1 536 tokens (MI355X, per forward: 1 025
  // tokens -5.6 %, one 1 100-token sequence -4.3 %, 8 x 160 -8.5 %, 5 x 300
  // -7.4 %, 3 x 512 -2.9 %, 3 x 600 -1.2 %, 6 x 200 + 100 -10 %): twice
  // the items fill more CUs, each with two waves per SIMD. One 2 048-token
  // sequence loses 2 % (its items' key runs halve: 2 of 32 tiles instead of
  // 5 of 13), so it keeps 128-row items. Between half a round and 0.6 of
  // a round, pairs only for ragged batches (the longest sequence at least
  // 1.25x the mean): one round of 128-row items takes as long as its
  // longest item, which the pairs halve while the short items fill their
  // partial second round (the C2 batch, 143 items, on one stream: 5.605 ->
  // 5.519 ms per forward, attention 1.13 -> 1.03 ms); with equal lengths
  // that second round is only added time (36 x 160: 5.39 -> 5.67, 43 x
  // 128: 5.21 -> 5.45 ms). From two rounds (C3, C5) the 128-row items stay
  // 20-30 % faster.
  if (p.any_tiles) {
    int64_t n8 = 0, sum_len = 0;
    int max_len = 0;
    for (int b = 0; b < in.B; b++) {
      n8 += ((int64_t)p.Gt * in.lengths[b] + 127) / 128 * p.hkv_t;
      max_len = std::max(max_len, (int)in.lengths[b]);
      sum_len += in.lengths[b];
    }
    const bool ragged = 4LL * max_len * in.B >= 5 * sum_len;
    if (in.groups > 1 && 2 * n8 > in.cus && 5 * n8 <= 3LL * in.cus) p.waves_t = 4;
    if (in.groups == 1 && max_len < 1536 && (2 * n8 <= in.cus || (ragged && 5 * n8 <= 3LL * in.cus)))
      p.waves_t = 4;
    if (in.forced_rows) p.waves_t = in.forced_rows / 16;
  }
  const int istep_t = 16 * p.waves_t;
  for (int b = 0; b < in.B; b++) {
    const int L = in.lengths[b];
    if (p.any_tiles) {
      p.n_items_t += ((int64_t)p.Gt * L + istep_t - 1) / istep_t * p.hkv_t;
      p.n_tiles += (L + in.tile_keys - 1) / in.tile_keys;
    }
    if (p.any_var) p.n_items_v += ((int64_t)L + in.varlen_qblock - 1) / in.varlen_qblock * in.H;
  }
  // Attention over few items (a short batch on one stream) cuts each
  // item's keys into up to eight runs of whole tiles, one workgroup each, so
  // that more CUs share the key loop: C1's 12 fp32 items (128 tokens, 3
  // heads) become 96 workgroups of one 16-key tile. Per forward on MI355X
  // against the earlier rule (at most four runs of at least two tiles):
  // 128 tokens 1.171 -> 1.140 ms, 64 1.071 -> 1.038, 200 1.380 -> 1.294,
  // 300 1.678 -> 1.584, 400 1.838 -> 1.760, 500 1.913 -> 1.900; 4 x 128
  // (runs capped at four by their length) unchanged; 32 tokens keep one run.
  if (p.any_var && in.groups == 1 && p.M <= in.split_rows && 2 * p.n_items_v <= in.cus) {
    p.kparts_v = (int)std::min<int64_t>(in.max_key_parts, in.cus / std::max<int64_t>(p.n_items_v, 1));
    const int tiles16 = (in.T + 15) / 16;  // the longest sequence's 16-key tiles
    p.kparts_v = std::max(1, std::min(p.kparts_v, tiles16));  // at least one tile per run
    // no more runs than its run length needs (8 tiles in 5 runs are runs of
    // 2, 2, 2, 2 and an empty one: 4 runs)
    const int per = (tiles16 + p.kparts_v - 1) / p.kparts_v;
    p.kparts_v = (tiles16 + per - 1) / per;
    if (in.T <= 32) p.kparts_v = 1;  // two tiles: the combine launch costs more than a tile
    if (in.forced_key_parts) p.kparts_v = in.forced_key_parts;
  }
  if (p.any_tiles) {
    // fewer tile items than CUs (one or two long sequences): each item's
    // key tiles are cut into runs of at least four, one workgroup each
    const int max_tiles = (in.T + in.tile_keys - 1) / in.tile_keys;
    if (p.n_items_t < in.cus) {
      p.kparts_t = (int)std::min<int64_t>(in.max_key_parts, in.cus / std::max<int64_t>(p.n_items_t, 1));
      p.kparts_t = std::max(1, std::min(p.kparts_t, max_tiles / 4));
    }
    if (in.forced_key_parts) p.kparts_t = std::min(in.forced_key_parts, max_tiles);
  }
}

namespace {

// Estimated time of a launch whose workgroup i (cost cost(i)) runs on XCD
// i % 8, each XCD's slots taking its workgroups in order as slots free up.
template <class Cost>
double launch_span(int64_t n, int slots, Cost cost) {
  const int per = std::max(1, slots / kXcds);
  std::vector<std::vector<double>> free_at(kXcds, std::vector<double>(per, 0.0));
  double span = 0;
  for (int64_t i = 0; i < n; i++) {
    auto& f = free_at[i % kXcds];
    auto it = std::min_element(f.begin(), f.end());
    *it += cost(i);
    span = std::max(span, *it);
  }
  return span;
}

}  // namespace

void plan_items(const AttnPlanIn& in, AttnPlan& p, int32_t* items, std::vector<int>& order) {
  // Work items of each group, longest sequences first: an item's work grows
  // with its sequence's length, and dispatching the long ones first
  // shortens the tail.
  int64_t it = 0;
  for (int list = 0; list < 2; list++) {
    const bool tiles = list == 0;
    if (!(tiles ? p.any_tiles : p.any_var)) continue;
    const int istep = tiles ? 16 * p.waves_t : in.varlen_qblock;
    const int iheads = tiles ? p.hkv_t : in.H;  // items per row block
    for (int gi = 0; gi < in.groups; gi++) {
      const int b0 = in.gb[gi], b1 = in.gb[gi + 1];
      order.resize(b1 - b0);
      for (int b = b0; b < b1; b++) order[b - b0] = b;
      std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return in.lengths[x] > in.lengths[y]; });
      const int64_t first = it;
      if (tiles ? p.kparts_t == 1 : p.kparts_v == 1) {
        // XCD-local items: workgroup i of a launch runs on XCD i % 8, and
        // every item of a sequence reads the same keys and values (the tile
        // path's images, the fp32 path's rows of q|k|v). Queue x of the
        // group's n items takes positions x, x + 8, ... : n / 8 of them,
        // plus one for x < n % 8. A sequence's items (sequences longest
        // first) fill the queue with the most room and move to the next
        // only when it is full, so its keys and values are fetched into as
        // few XCD L2s as the balance allows; each queue ends exactly full.
        int64_t n = 0;
        for (int b : order) n += ((int64_t)(tiles ? p.Gt : 1) * in.lengths[b] + istep - 1) / istep * iheads;
        std::vector<std::vector<int64_t>> q(kXcds);  // packed (sequence, first row, head)
        std::vector<int64_t> room(kXcds);
        for (int x = 0; x < kXcds; x++) room[x] = n / kXcds + (x < n % kXcds ? 1 : 0);
        for (int b : order) {
          const int rows_b = tiles ? p.Gt * in.lengths[b] : in.lengths[b];
          int x = -1;
          for (int q0 = 0; q0 < rows_b; q0 += istep)
            for (int h = 0; h < iheads; h++) {
              if (x < 0 || room[x] == 0) {
                x = 0;
                for (int y = 1; y < kXcds; y++)
                  if (room[y] > room[x]) x = y;
              }
              q[x].push_back(((int64_t)b << 32) | ((int64_t)q0 << 8) | h);
              room[x]--;
            }
        }
        // Equal item counts per XCD are not equal work when sequence lengths
        // differ and the launch takes more than one round: keep this order
        // only where its estimated span (an item costs its key tiles plus
        // two for its prologue; one workgroup per CU, as the tile attention
        // and the head_dim-512 fp32 kernel run) is within 3 % of the plain
        // longest-first order's (C4 on
        // one stream: 281 items of 1 024-2 048 tokens, +14 % measured for
        // the attention with XCD-local queues; C3, equal lengths: -4.7 %).
        const int keys = tiles ? in.tile_keys : 16;
        auto cost_of = [&](int b) { return 2.0 + (double)((in.lengths[b] + keys - 1) / keys); };
        std::vector<int32_t> plain;
        for (int b : order) {
          const int rows_b = tiles ? p.Gt * in.lengths[b] : in.lengths[b];
          for (int q0 = 0; q0 < rows_b; q0 += istep)
            for (int h = 0; h < iheads; h++) plain.push_back(b);
        }
        // and only for long key loops (a group's mean length at least 12
        // key tiles of 32): C3's 512-token sequences -1.7 % per forward
        // (attention -4 %), while C2's micro-batches (mean 172 tokens) ran
        // 0.7 % slower with the XCD-local order and C5 (mean 72) equal,
        // though it cut the C2 launch's HBM fetch of the images 2.7 times
        // (the spans are estimated only where that rule leaves a choice)
        int64_t keys_sum = 0;
        for (int b : order) keys_sum += in.lengths[b];
        const bool long_keys = keys_sum >= 384LL * (int64_t)order.size();
        bool local = long_keys;
        if (long_keys && !in.forced_xcd) {
          const int slots = in.cus;
          const double span_plain = launch_span(n, slots, [&](int64_t i) { return cost_of(plain[i]); });
          const double span_xcd =
              launch_span(n, slots, [&](int64_t i) { return cost_of((int)(q[i % kXcds][i / kXcds] >> 32)); });
          local = span_xcd <= 1.03 * span_plain;
        }
        if (in.forced_xcd) local = in.forced_xcd > 0;
        for (int64_t i = 0; i < n; i++) {
          if (local) {
            const int64_t e = q[i % kXcds][i / kXcds];
            items[3 * it] = (int32_t)(e >> 32);
            items[3 * it + 1] = (int32_t)((e >> 8) & 0xFFFFFF);
            items[3 * it + 2] = (int32_t)(e & 0xFF);
          } else {
            items[3 * it] = plain[i];
          }
          it++;
        }
        if (!local) {  // the plain order's rows and heads
          it -= n;
          for (int b : order) {
            const int rows_b = tiles ? p.Gt * in.lengths[b] : in.lengths[b];
            for (int q0 = 0; q0 < rows_b; q0 += istep)
              for (int h = 0; h < iheads; h++) {
                items[3 * it + 1] = q0;
                items[3 * it + 2] = h;
                it++;
              }
          }
        }
        (tiles ? p.xcd_local_t : p.xcd_local_v)[gi] = local;
      } else {
        for (int b : order) {
          const int rows_b = tiles ? p.Gt * in.lengths[b] : in.lengths[b];
          for (int q0 = 0; q0 < rows_b; q0 += istep) {
            for (int h = 0; h < iheads; h++) {
              items[3 * it] = b;
              items[3 * it + 1] = q0;
              items[3 * it + 2] = h;
              it++;
            }
          }
        }
      }
      (tiles ? p.group_items_t : p.group_items_v)[gi] = it - first;
    }
  }
}

}  // namespace fa
