// KV-block placement policy: which logical blocks sit in VRAM (tier 0), host RAM (1) or
// the spill tier (2). Restates pager/src/core.rs and pager/src/metrics.rs of the reference
// in C++17; compiled with -ffp-contract=off so every f32 expression rounds exactly as the
// Rust code does (Rust never fuses multiply-add).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace pgr {

enum class Tier : uint8_t { Vram = 0, Ram = 1, Ssd = 2 };
enum class Policy : int { RecentOnly = 0, SinksRecent = 1, HeavyHitter = 2, SinksHeavyHitter = 3 };

// core.rs:24-33: unknown names fall back to heavy_hitter.
Policy policy_from_name(const std::string& name);

// metrics.rs:4-27.
struct PagerMetrics {
  uint64_t tokens = 0;
  uint64_t vram_peak = 0;
  uint64_t ram_peak = 0;
  uint64_t swap_vram_ram = 0;
  uint64_t swap_ram_ssd = 0;
  double attention_mass_total = 0.0;
  double attention_mass_vram = 0.0;
};

class PlacementPager {
 public:
  static constexpr uint64_t kBlockSizeBytes = 16ull * 1024 * 1024;  // core.rs:6 (logical block)
  static constexpr uint64_t kSinkBlocks = 4;                        // core.rs:7

  PlacementPager(uint64_t vram, uint64_t ram, uint64_t recent_window, uint64_t rebalance_interval,
                 float promote_margin, float ram_promote_margin, Policy policy);

  // core.rs:87-98. Returns false (state unchanged past the point of failure) when
  // rebalance_interval is 0 and a rebalance check needs it, mirroring Rust's panic.
  bool on_step(uint64_t token_idx, const float* attention, size_t n);
  // core.rs:100-107.
  void force_rebalance(uint64_t token_idx);

  size_t num_blocks() const { return blocks_.size(); }
  void tiers(uint8_t* out) const;             // core.rs:113-122
  size_t vram_block_ids(uint64_t* out) const;  // core.rs:124-130; returns the count
  size_t vram_count() const;
  const PagerMetrics& metrics() const { return metrics_; }

 private:
  struct Block {
    uint64_t id;
    uint64_t size;
    float score;
    Tier tier;
    bool pinned;
  };

  void ensure_blocks(size_t count);
  void update_scores(const float* attention, size_t n);
  void update_attention_quality(const float* attention, size_t n);
  void pin_blocks(uint64_t token_idx);
  void place_blocks();
  void place_baseline(const std::vector<Tier>& old, size_t max_vram, size_t max_ram);
  void place_heavy_hitter(const std::vector<Tier>& old, size_t max_vram, size_t max_ram);
  void place_sinks_heavy_hitter(const std::vector<Tier>& old, size_t max_vram, size_t max_ram);
  void assign_ranked(const std::vector<size_t>& ranked, size_t max_vram, size_t max_ram);
  void reset_tiers(Tier t);
  void enforce_vram_budget_keep_best(size_t max_vram);
  void promote_vram_with_hysteresis(size_t max_vram);
  void fill_ram(size_t max_ram);
  void trim_ram(size_t max_ram);
  void promote_ram_with_hysteresis(size_t max_ram);
  long worst_unpinned_vram() const;
  long best_non_vram() const;
  long worst_ram() const;
  long best_ssd() const;
  void count_tier_changes(const std::vector<Tier>& old);
  void update_memory_peaks();

  uint64_t vram_;
  uint64_t ram_;
  uint64_t recent_window_;
  uint64_t rebalance_interval_;
  float promote_margin_;
  float ram_promote_margin_;
  Policy policy_;
  PagerMetrics metrics_;
  std::vector<Block> blocks_;
};

}  // namespace pgr
