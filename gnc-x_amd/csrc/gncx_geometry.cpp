// gncx_geometry.cpp -- the loader's layer-coordinate and slot bookkeeping.
//
// Two pieces of host arithmetic the streamer calls once at load time
// (lua/gncx_streamer.lua:502-564): the centre-relative coordinate of a layer
// (csrc/gncx_genome_vm.hpp:35-60) and the diagonal slot manager that picks
// the colour (k, d, R) of each KV-cache buffer (csrc/gncx_geometric_mm.hpp).
// Neither touches the GPU.  The observable results -- the coordinate fields,
// and which (k, d, R, index) each allocation returns, the used / capacity
// counts and the fragmentation figure after any sequence of calls -- are the
// reference's; the state is kept as one 64-bit occupancy word and eight 8-bit
// diagonal words per 64-frame grid.
#include <algorithm>
#include <bit>
#include <cstdint>
#include <cstdlib>

#include "../../include/gncx_llm_core.h"

#define GNCX_API extern "C" __attribute__((visibility("default")))

namespace {

// odd rotation factors, coprime with 8 (gncx_geometric_mm.hpp:28)
constexpr uint8_t kRot[4] = {1, 3, 5, 7};

// frame of (k, d) inside an 8 x 8 grid: row (d + k R) mod 8, column
// (d R + k) mod 8 with R = kRot[k mod 4] (gncx_geometric_mm.hpp:31-37, 47-50)
uint32_t frame_of(uint8_t k, uint8_t d) {
    const uint32_t r = kRot[k & 3u];
    const uint32_t row = (d + static_cast<uint32_t>(k) * r) & 7u;
    const uint32_t col = ((static_cast<uint32_t>(d) * r) & 7u) + k;
    return row * 8u + (col & 7u);
}

class SlotGrids {
  public:
    static constexpr uint32_t kFrames = 64;
    static constexpr uint32_t kMaxGrids = 8;

    explicit SlotGrids(uint32_t min_frames) {
        grids_ = std::clamp((min_frames + kFrames - 1) / kFrames, 1u, kMaxGrids);
    }

    // gncx_geometric_mm.hpp:83-108.  Grid by grid, diagonals d = 0..7 whose
    // word (index d R mod 8) is not full are searched at d, d+1, ... (mod 8)
    // for the first free frame; the word records the offset used.
    bool alloc(uint8_t k, uint8_t& d_out, uint8_t& r_out, uint32_t& index) {
        const uint8_t r = kRot[k & 3u];
        for (uint32_t g = 0; g < grids_; ++g) {
            for (uint32_t d = 0; d < 8; ++d) {
                uint8_t& diag = diag_[g][(d * r) & 7u];
                if (diag == 0xff) continue;
                for (uint32_t off = 0; off < 8; ++off) {
                    const uint8_t dd = static_cast<uint8_t>((d + off) & 7u);
                    const uint32_t f = frame_of(k, dd);
                    if (used_[g] >> f & 1u) continue;
                    used_[g] |= uint64_t{1} << f;
                    diag |= static_cast<uint8_t>(1u << off);
                    d_out = dd;
                    r_out = r;
                    index = g * kFrames + f;
                    return true;
                }
            }
        }
        return false;
    }

    // gncx_geometric_mm.hpp:111-124.  Clears the frame and the lowest bit of
    // the diagonal word of (k, d); indices past the grids are ignored.
    void release(uint8_t k, uint8_t d, uint32_t index) {
        const uint32_t g = index / kFrames;
        if (g >= grids_) return;
        used_[g] &= ~(uint64_t{1} << (index % kFrames));
        uint8_t& diag = diag_[g][(static_cast<uint32_t>(d) * kRot[k & 3u]) & 7u];
        diag = static_cast<uint8_t>(diag & (diag - 1u));
    }

    // gncx_geometric_mm.hpp:127-146: 1 - (longest free run) / (free frames),
    // frames taken in index order across grids; 0 when nothing is free.
    float fragmentation() const {
        uint32_t free_frames = 0, run = 0, best = 0;
        for (uint32_t g = 0; g < grids_; ++g) {
            for (uint32_t f = 0; f < kFrames; ++f) {
                if (used_[g] >> f & 1u) {
                    best = std::max(best, run);
                    run = 0;
                } else {
                    ++free_frames;
                    ++run;
                }
            }
        }
        best = std::max(best, run);
        if (free_frames == 0) return 0.0f;
        return 1.0f - static_cast<float>(best) / static_cast<float>(free_frames);
    }

    size_t used() const {
        size_t n = 0;
        for (uint32_t g = 0; g < grids_; ++g) n += static_cast<size_t>(std::popcount(used_[g]));
        return n;
    }

    size_t capacity() const { return static_cast<size_t>(grids_) * kFrames; }

  private:
    uint32_t grids_ = 1;
    uint64_t used_[kMaxGrids] = {};
    uint8_t diag_[kMaxGrids][8] = {};
};

}  // namespace

// cpp:672-686 with gncx_genome_vm.hpp:35-60: origin = max(1, total) / 2,
// rel = layer - origin, hemisphere 0 when rel >= 0; the sieve order grows
// from 2 at the centre to 4 at the edges (2 + 2 |rel| / origin, clamped), or
// is base_k clamped to [1, 4] when the origin is 0.
GNCX_API void gncx_genome_get_layer_coordinate(int32_t layer_index, int32_t total_layers, int32_t base_k,
                                               int32_t* out_rel_layer, int32_t* out_dist_centro,
                                               int32_t* out_crivo_k, int32_t* out_hemisferio) {
    const int32_t origin = std::max<int32_t>(1, total_layers) / 2;
    const int32_t rel = layer_index - origin;
    const int32_t dist = std::abs(rel);
    const int32_t k = origin > 0 ? std::clamp(2 + dist * 2 / origin, 2, 4) : std::clamp(base_k, 1, 4);
    if (out_rel_layer) *out_rel_layer = rel;
    if (out_dist_centro) *out_dist_centro = dist;
    if (out_crivo_k) *out_crivo_k = k;
    if (out_hemisferio) *out_hemisferio = rel >= 0 ? 0 : 1;
}

// cpp:2059-2111
GNCX_API void* gncx_geo_mm_create(uint32_t min_frames) { return new SlotGrids(min_frames); }

GNCX_API void gncx_geo_mm_destroy(void* handle) { delete static_cast<SlotGrids*>(handle); }

GNCX_API int32_t gncx_geo_alloc(void* handle, uint8_t k_hint, uint8_t* out_k, uint8_t* out_d, uint8_t* out_R,
                                uint32_t* out_linear_idx) {
    if (!handle) return 0;
    uint8_t d = 0, r = 0;
    uint32_t index = 0;
    if (!static_cast<SlotGrids*>(handle)->alloc(k_hint, d, r, index)) return 0;
    if (out_k) *out_k = k_hint;
    if (out_d) *out_d = d;
    if (out_R) *out_R = r;
    if (out_linear_idx) *out_linear_idx = index;
    return 1;
}

GNCX_API void gncx_geo_free(void* handle, uint8_t k, uint8_t d, uint8_t R, uint32_t linear_idx) {
    (void)R;  // the reference recomputes the rotation from k (gncx_geometric_mm.hpp:117)
    if (handle) static_cast<SlotGrids*>(handle)->release(k, d, linear_idx);
}

GNCX_API float gncx_geo_fragmentation(void* handle) {
    return handle ? static_cast<SlotGrids*>(handle)->fragmentation() : 0.0f;
}

GNCX_API size_t gncx_geo_used(void* handle) { return handle ? static_cast<SlotGrids*>(handle)->used() : 0; }

GNCX_API size_t gncx_geo_capacity(void* handle) {
    return handle ? static_cast<SlotGrids*>(handle)->capacity() : 0;
}
