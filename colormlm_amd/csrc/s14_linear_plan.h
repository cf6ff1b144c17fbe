// Launch planning of the FAST fp8_linear (k_linear_fast): how many 128-k
// chunks each wavefront streams (its K split is groups / cw) and how many
// 32-token blocks one launch takes, so that the split-K partials and the
// arrival counters always fit the context's linear workspace.  Plain C++ (no
// HIP types): the library and a host-only test include it.
#pragma once

#include <cstddef>
#include <cstdint>

namespace s14 {

constexpr uint32_t kLinGroup = 128;                 // k values per activation / weight scale (fp8.py:14)
constexpr uint32_t kLinTile = 32;                   // FAST: output rows (and token columns) per MFMA tile
constexpr size_t kLinPartBytes = size_t(32) << 20;  // FAST split-K partials (per context)
constexpr uint32_t kLinMaxCounters = 65536;         // FAST: one arrival counter per (row tile, token block)
// Staged activations per wavefront: ntok x cw chunks x 128 bf16, plus the
// f32 scale of every (token, chunk) when the scales are f32.
constexpr uint32_t kLinStageBytes = 40u * 1024u;
// Wavefronts a FAST launch aims for (more K splits fill the GPU for short,
// wide weights; fewer amortise the ring's prologue).
constexpr uint32_t kLinFastWaves = 1024;

constexpr uint32_t lin_stage_bytes(uint32_t ntok, uint32_t cw) { return ntok * cw * (kLinGroup * 2u + 4u); }

// Bytes of split-K partials a launch of `blocks` token blocks writes.
constexpr uint64_t lin_part_bytes(uint32_t tiles, uint32_t blocks, uint32_t splits) {
  return splits > 1u ? uint64_t(tiles) * blocks * splits * kLinTile * kLinTile * sizeof(float) : 0u;
}

// Chunks per wavefront for one launch of `blocks` token blocks: the smallest
// multiple of 4 dividing G that keeps the grid within kLinFastWaves
// wavefronts, else the largest that fits.  A width fits when its staged
// activations fit kLinStageBytes and, if it splits K, the launch's partials
// fit kLinPartBytes and its (tile, block) counters kLinMaxCounters.  0: no
// width fits.
inline uint32_t lin_fast_chunks(uint32_t G, uint32_t tiles, uint32_t blocks, uint32_t ntok) {
  const uint64_t tiles_all = uint64_t(tiles) * blocks;
  uint32_t best = 0;
  for (uint32_t cw = 4; cw <= G; cw += 4) {
    if (G % cw) continue;
    if (lin_stage_bytes(ntok, cw) > kLinStageBytes) break;
    const uint32_t splits = G / cw;
    if (splits > 1u && (tiles_all > kLinMaxCounters || lin_part_bytes(tiles, blocks, splits) > kLinPartBytes))
      continue;
    best = cw;
    if (tiles_all * splits <= kLinFastWaves) return cw;
  }
  return best;
}

struct LinFastPlan {
  uint32_t cw;      // chunks per wavefront; 0: FAST cannot take the shape
  uint32_t blocks;  // 32-token blocks per launch (the last launch may take fewer)
};

// The launch plan for m tokens: all token blocks in one launch when a chunk
// width fits them, else halved until one does.  {0, 0} when no width fits
// even one block (G not a multiple of 4, or K split so finely that one
// block's partials exceed the workspace): the caller takes the EXACT path.
inline LinFastPlan lin_fast_plan(uint32_t m, uint32_t n, uint32_t G) {
  if (m == 0 || n == 0 || G == 0 || G % 4u) return {0, 0};
  const uint32_t tiles = (n + kLinTile - 1) / kLinTile;
  const uint32_t ntok = m < kLinTile ? m : kLinTile;
  uint32_t blocks = (m + kLinTile - 1) / kLinTile;
  for (;;) {
    if (const uint32_t cw = lin_fast_chunks(G, tiles, blocks, ntok)) return {cw, blocks};
    if (blocks == 1) return {0, 0};
    blocks = (blocks + 1) / 2;
  }
}

}  // namespace s14
