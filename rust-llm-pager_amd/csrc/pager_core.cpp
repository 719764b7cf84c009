// Placement policy, restated from pager/src/core.rs. Ordering rules that decide ties:
//  * every sort is stable (Rust slice::sort_by) -> std::stable_sort;
//  * Iterator::min_by keeps the first of equal minima, max_by returns the last of equal
//    maxima (core.rs:479-513) -> explicit folds below;
//  * scores compare with partial_cmp and NaN counts as Equal (core.rs:553-555).
#include "pager_core.h"

#include <algorithm>
#include <unordered_set>

namespace pgr {

namespace {

// core.rs:553-555. -1 less, 0 equal (incl. NaN), 1 greater.
inline int compare_scores(float a, float b) {
  if (a < b) return -1;
  if (a > b) return 1;
  return 0;
}

}  // namespace

Policy policy_from_name(const std::string& name) {
  if (name == "recent_only") return Policy::RecentOnly;
  if (name == "sinks_recent") return Policy::SinksRecent;
  if (name == "heavy_hitter") return Policy::HeavyHitter;
  if (name == "sinks_heavy_hitter") return Policy::SinksHeavyHitter;
  return Policy::HeavyHitter;
}

PlacementPager::PlacementPager(uint64_t vram, uint64_t ram, uint64_t recent_window, uint64_t rebalance_interval,
                               float promote_margin, float ram_promote_margin, Policy policy)
    : vram_(vram),
      ram_(ram),
      recent_window_(recent_window),
      rebalance_interval_(rebalance_interval),
      promote_margin_(promote_margin),
      ram_promote_margin_(ram_promote_margin),
      policy_(policy) {}

bool PlacementPager::on_step(uint64_t token_idx, const float* attention, size_t n) {
  metrics_.tokens += 1;
  ensure_blocks(n);
  update_scores(attention, n);
  update_attention_quality(attention, n);
  pin_blocks(token_idx);
  if (metrics_.tokens == 1) {
    force_rebalance(token_idx);
    return true;
  }
  if (rebalance_interval_ == 0) return false;  // Rust: remainder with a divisor of zero
  if (metrics_.tokens % rebalance_interval_ == 0) force_rebalance(token_idx);
  return true;
}

void PlacementPager::force_rebalance(uint64_t token_idx) {
  ensure_blocks(static_cast<size_t>(token_idx) + 1);
  pin_blocks(token_idx);
  place_blocks();
  update_memory_peaks();
}

void PlacementPager::tiers(uint8_t* out) const {
  for (size_t i = 0; i < blocks_.size(); ++i) out[i] = static_cast<uint8_t>(blocks_[i].tier);
}

size_t PlacementPager::vram_block_ids(uint64_t* out) const {
  size_t c = 0;
  for (const Block& b : blocks_)
    if (b.tier == Tier::Vram) {
      if (out) out[c] = b.id;
      ++c;
    }
  return c;
}

size_t PlacementPager::vram_count() const { return vram_block_ids(nullptr); }

void PlacementPager::ensure_blocks(size_t count) {
  if (blocks_.size() >= count) return;
  blocks_.reserve(count);
  while (blocks_.size() < count) {
    const uint64_t id = blocks_.size();
    blocks_.push_back(Block{id, kBlockSizeBytes, 0.0f, Tier::Ram, false});
  }
}

void PlacementPager::update_scores(const float* attention, size_t n) {
  // core.rs:145-149: f32 EMA, two products then a sum, each rounded to f32.
  const size_t m = std::min(n, blocks_.size());
  for (size_t i = 0; i < m; ++i) {
    const float decayed = blocks_[i].score * 0.90f;
    const float fresh = attention[i] * 0.10f;
    blocks_[i].score = decayed + fresh;
  }
}

void PlacementPager::update_attention_quality(const float* attention, size_t n) {
  // core.rs:151-165: f64 sums; VRAM share uses the tiers from before this step's placement.
  double total = 0.0, vram = 0.0;
  const size_t m = std::min(n, blocks_.size());
  for (size_t i = 0; i < m; ++i) {
    const double s = static_cast<double>(attention[i]);
    total += s;
    if (blocks_[i].tier == Tier::Vram) vram += s;
  }
  metrics_.attention_mass_total += total;
  metrics_.attention_mass_vram += vram;
}

void PlacementPager::pin_blocks(uint64_t token_idx) {
  // core.rs:167-181
  const uint64_t recent_start = token_idx > recent_window_ ? token_idx - recent_window_ : 0;
  for (Block& b : blocks_) {
    const bool is_recent = b.id >= recent_start;
    const bool is_sink = b.id < kSinkBlocks;
    b.pinned = policy_ == Policy::RecentOnly ? is_recent : (is_recent || is_sink);
  }
}

void PlacementPager::place_blocks() {
  // core.rs:183-199
  std::vector<Tier> old(blocks_.size());
  for (size_t i = 0; i < blocks_.size(); ++i) old[i] = blocks_[i].tier;
  const size_t max_vram = static_cast<size_t>(vram_ / kBlockSizeBytes);
  const size_t max_ram = static_cast<size_t>(ram_ / kBlockSizeBytes);
  switch (policy_) {
    case Policy::RecentOnly:
    case Policy::SinksRecent:
      place_baseline(old, max_vram, max_ram);
      break;
    case Policy::HeavyHitter:
      place_heavy_hitter(old, max_vram, max_ram);
      break;
    case Policy::SinksHeavyHitter:
      place_sinks_heavy_hitter(old, max_vram, max_ram);
      break;
  }
}

void PlacementPager::place_baseline(const std::vector<Tier>& old, size_t max_vram, size_t max_ram) {
  // core.rs:201-219: rank by (pinned desc, id asc).
  std::vector<size_t> ranked(blocks_.size());
  for (size_t i = 0; i < ranked.size(); ++i) ranked[i] = i;
  std::stable_sort(ranked.begin(), ranked.end(), [this](size_t a, size_t b) {
    if (blocks_[a].pinned != blocks_[b].pinned) return blocks_[a].pinned;
    return blocks_[a].id < blocks_[b].id;
  });
  reset_tiers(Tier::Ssd);
  assign_ranked(ranked, max_vram, max_ram);
  count_tier_changes(old);
}

void PlacementPager::place_heavy_hitter(const std::vector<Tier>& old, size_t max_vram, size_t max_ram) {
  // core.rs:221-255
  bool has_vram = false;
  for (const Block& b : blocks_) has_vram = has_vram || b.tier == Tier::Vram;
  if (!has_vram) {
    std::vector<size_t> ranked(blocks_.size());
    for (size_t i = 0; i < ranked.size(); ++i) ranked[i] = i;
    std::stable_sort(ranked.begin(), ranked.end(), [this](size_t a, size_t b) {
      if (blocks_[a].pinned != blocks_[b].pinned) return blocks_[a].pinned;
      return compare_scores(blocks_[b].score, blocks_[a].score) < 0;  // score desc
    });
    assign_ranked(ranked, max_vram, max_ram);
    count_tier_changes(old);
    return;
  }
  for (Block& b : blocks_)
    if (b.pinned) b.tier = Tier::Vram;
  enforce_vram_budget_keep_best(max_vram);
  promote_vram_with_hysteresis(max_vram);
  fill_ram(max_ram);
  promote_ram_with_hysteresis(max_ram);
  count_tier_changes(old);
}

void PlacementPager::place_sinks_heavy_hitter(const std::vector<Tier>& old, size_t max_vram, size_t max_ram) {
  // core.rs:257-318
  reset_tiers(Tier::Ssd);
  if (max_vram == 0) {
    count_tier_changes(old);
    return;
  }
  std::unordered_set<uint64_t> selected;
  const size_t n = blocks_.size();
  for (size_t i = 0; i < n && i < kSinkBlocks; ++i) {
    if (selected.size() >= max_vram) break;
    selected.insert(blocks_[i].id);
  }
  const size_t remaining = max_vram > selected.size() ? max_vram - selected.size() : 0;
  const size_t half = std::max<size_t>(max_vram / 2, 1);
  const size_t recent_budget =
      std::min<size_t>(std::min<size_t>(static_cast<size_t>(recent_window_), half), remaining);
  const size_t recent_start = n > recent_budget ? n - recent_budget : 0;
  for (size_t i = recent_start; i < n; ++i) {
    if (selected.size() >= max_vram) break;
    selected.insert(blocks_[i].id);
  }
  std::vector<size_t> scored;
  for (size_t i = 0; i < n; ++i)
    if (!selected.count(blocks_[i].id)) scored.push_back(i);
  std::stable_sort(scored.begin(), scored.end(),
                   [this](size_t a, size_t b) { return compare_scores(blocks_[b].score, blocks_[a].score) < 0; });
  for (size_t i : scored) {
    if (selected.size() >= max_vram) break;
    selected.insert(blocks_[i].id);
  }
  for (Block& b : blocks_)
    if (selected.count(b.id)) b.tier = Tier::Vram;
  fill_ram(max_ram);
  count_tier_changes(old);
}

void PlacementPager::assign_ranked(const std::vector<size_t>& ranked, size_t max_vram, size_t max_ram) {
  // core.rs:320-335
  for (size_t rank = 0; rank < ranked.size(); ++rank) {
    Tier t = Tier::Ssd;
    if (rank < max_vram)
      t = Tier::Vram;
    else if (rank < max_vram + max_ram)
      t = Tier::Ram;
    blocks_[ranked[rank]].tier = t;
  }
}

void PlacementPager::reset_tiers(Tier t) {
  for (Block& b : blocks_) b.tier = t;
}

void PlacementPager::enforce_vram_budget_keep_best(size_t max_vram) {
  // core.rs:343-366
  std::vector<size_t> ids;
  for (size_t i = 0; i < blocks_.size(); ++i)
    if (blocks_[i].tier == Tier::Vram) ids.push_back(i);
  if (ids.size() <= max_vram) return;
  std::stable_sort(ids.begin(), ids.end(), [this](size_t a, size_t b) {
    if (blocks_[a].pinned != blocks_[b].pinned) return blocks_[a].pinned;
    return compare_scores(blocks_[b].score, blocks_[a].score) < 0;
  });
  for (size_t k = max_vram; k < ids.size(); ++k) blocks_[ids[k]].tier = Tier::Ram;
}

long PlacementPager::worst_unpinned_vram() const {
  // min_by: the running minimum is replaced only by a strictly smaller score.
  long best = -1;
  for (size_t i = 0; i < blocks_.size(); ++i) {
    const Block& b = blocks_[i];
    if (b.tier != Tier::Vram || b.pinned) continue;
    if (best < 0 || compare_scores(blocks_[best].score, b.score) > 0) best = static_cast<long>(i);
  }
  return best;
}

long PlacementPager::best_non_vram() const {
  // max_by: the running maximum is replaced unless it is strictly greater.
  long best = -1;
  for (size_t i = 0; i < blocks_.size(); ++i) {
    const Block& b = blocks_[i];
    if (b.tier == Tier::Vram) continue;
    if (best < 0 || compare_scores(blocks_[best].score, b.score) <= 0) best = static_cast<long>(i);
  }
  return best;
}

long PlacementPager::worst_ram() const {
  long best = -1;
  for (size_t i = 0; i < blocks_.size(); ++i) {
    const Block& b = blocks_[i];
    if (b.tier != Tier::Ram) continue;
    if (best < 0 || compare_scores(blocks_[best].score, b.score) > 0) best = static_cast<long>(i);
  }
  return best;
}

long PlacementPager::best_ssd() const {
  long best = -1;
  for (size_t i = 0; i < blocks_.size(); ++i) {
    const Block& b = blocks_[i];
    if (b.tier != Tier::Ssd) continue;
    if (best < 0 || compare_scores(blocks_[best].score, b.score) <= 0) best = static_cast<long>(i);
  }
  return best;
}

void PlacementPager::promote_vram_with_hysteresis(size_t max_vram) {
  // core.rs:368-400. The iteration cap only matters for NaN scores, where the Rust loop
  // can swap forever; for ordered scores each swap strictly raises the VRAM score sum.
  const size_t cap = blocks_.size() * blocks_.size() + 16;
  for (size_t iter = 0; iter < cap; ++iter) {
    size_t vram_count = 0;
    for (const Block& b : blocks_) vram_count += b.tier == Tier::Vram;
    if (vram_count < max_vram) {
      const long best = best_non_vram();
      if (best >= 0) {
        blocks_[best].tier = Tier::Vram;
        continue;
      }
      break;
    }
    const long worst = worst_unpinned_vram();
    if (worst < 0) break;
    const long best = best_non_vram();
    if (best < 0) break;
    const float improvement = blocks_[best].score - blocks_[worst].score;
    if (improvement <= promote_margin_) break;
    const Tier previous = blocks_[best].tier;
    blocks_[best].tier = Tier::Vram;
    blocks_[worst].tier = previous;
  }
}

void PlacementPager::fill_ram(size_t max_ram) {
  // core.rs:402-427
  size_t current = 0;
  for (const Block& b : blocks_) current += b.tier == Tier::Ram;
  if (current >= max_ram) {
    trim_ram(max_ram);
    return;
  }
  std::vector<size_t> cand;
  for (size_t i = 0; i < blocks_.size(); ++i)
    if (blocks_[i].tier == Tier::Ssd) cand.push_back(i);
  std::stable_sort(cand.begin(), cand.end(),
                   [this](size_t a, size_t b) { return compare_scores(blocks_[b].score, blocks_[a].score) < 0; });
  const size_t take = std::min(cand.size(), max_ram - current);
  for (size_t k = 0; k < take; ++k) blocks_[cand[k]].tier = Tier::Ram;
}

void PlacementPager::trim_ram(size_t max_ram) {
  // core.rs:429-448
  std::vector<size_t> ids;
  for (size_t i = 0; i < blocks_.size(); ++i)
    if (blocks_[i].tier == Tier::Ram) ids.push_back(i);
  if (ids.size() <= max_ram) return;
  std::stable_sort(ids.begin(), ids.end(),
                   [this](size_t a, size_t b) { return compare_scores(blocks_[a].score, blocks_[b].score) < 0; });
  const size_t overflow = ids.size() - max_ram;
  for (size_t k = 0; k < overflow; ++k) blocks_[ids[k]].tier = Tier::Ssd;
}

void PlacementPager::promote_ram_with_hysteresis(size_t max_ram) {
  // core.rs:450-477
  const size_t cap = blocks_.size() * blocks_.size() + 16;
  for (size_t iter = 0; iter < cap; ++iter) {
    size_t ram_count = 0;
    for (const Block& b : blocks_) ram_count += b.tier == Tier::Ram;
    if (ram_count < max_ram) break;
    const long worst = worst_ram();
    if (worst < 0) break;
    const long best = best_ssd();
    if (best < 0) break;
    const float improvement = blocks_[best].score - blocks_[worst].score;
    if (improvement <= ram_promote_margin_) break;
    blocks_[best].tier = Tier::Ram;
    blocks_[worst].tier = Tier::Ssd;
  }
}

void PlacementPager::count_tier_changes(const std::vector<Tier>& old) {
  // core.rs:515-531
  const size_t n = std::min(old.size(), blocks_.size());
  for (size_t i = 0; i < n; ++i) {
    const Tier a = old[i], b = blocks_[i].tier;
    const uint64_t sz = blocks_[i].size;
    const bool vr = (a == Tier::Vram && b == Tier::Ram) || (a == Tier::Ram && b == Tier::Vram);
    const bool rs = (a == Tier::Ram && b == Tier::Ssd) || (a == Tier::Ssd && b == Tier::Ram);
    const bool vs = (a == Tier::Vram && b == Tier::Ssd) || (a == Tier::Ssd && b == Tier::Vram);
    if (vr) metrics_.swap_vram_ram += sz;
    if (rs) metrics_.swap_ram_ssd += sz;
    if (vs) {
      metrics_.swap_vram_ram += sz;
      metrics_.swap_ram_ssd += sz;
    }
  }
}

void PlacementPager::update_memory_peaks() {
  // core.rs:533-550
  uint64_t vram_used = 0, ram_used = 0;
  for (const Block& b : blocks_) {
    if (b.tier == Tier::Vram) vram_used += b.size;
    if (b.tier == Tier::Ram) ram_used += b.size;
  }
  metrics_.vram_peak = std::max(metrics_.vram_peak, vram_used);
  metrics_.ram_peak = std::max(metrics_.ram_peak, ram_used);
}

}  // namespace pgr
