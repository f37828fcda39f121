// ring.cpp -- host-side slot bookkeeping of the 3-tier KV ring, the part of
// DynamicRingBuffer (src/ring_buffer.zig:7-147) that drives the device
// caches: slot numbering, activation clocks, and the active-slot list each
// token attends over.  K/V values themselves live in the model's HBM caches.
#include <string.h>

#include <vector>

#include "runtime.hpp"

using gh::fail;

struct gh_ring {
  size_t num_layers, num_anchors, window_size, num_recall, total_slots;
  std::vector<uint64_t> clocks;
  std::vector<uint8_t> active;
  uint64_t total_ingested = 0;
  size_t recall_start() const { return num_anchors + window_size; }
};

extern "C" {

gh_status gh_ring_create(uint32_t num_layers, uint32_t num_anchors, uint32_t window_size,
                         uint32_t num_recall, gh_ring** out) {
  if (!out) return fail(GH_ERR_INVALID, "gh_ring_create: out is null");
  *out = nullptr;
  if (num_layers == 0 || window_size == 0)
    return fail(GH_ERR_INVALID, "gh_ring_create: num_layers and window_size must be positive");
  gh_ring* r = new gh_ring();
  r->num_layers = num_layers;
  r->num_anchors = num_anchors;
  r->window_size = window_size;
  r->num_recall = num_recall;
  r->total_slots = (size_t)num_anchors + window_size + num_recall;  // ring_buffer.zig:23
  r->clocks.assign(r->num_layers * r->total_slots, 0);
  r->active.assign(r->num_layers * r->total_slots, 0);
  *out = r;
  return GH_OK;
}

void gh_ring_destroy(gh_ring* r) { delete r; }

uint32_t gh_ring_total_slots(const gh_ring* r) { return r ? (uint32_t)r->total_slots : 0; }

// getSlotIndex (ring_buffer.zig:56-59)
uint32_t gh_ring_slot_index(const gh_ring* r, uint64_t clock) {
  if (clock < r->num_anchors) return (uint32_t)clock;
  return (uint32_t)(r->num_anchors + (clock - r->num_anchors) % r->window_size);
}

// activateSlot (ring_buffer.zig:61-68); writeKV's bookkeeping is the same.
uint32_t gh_ring_activate_slot(gh_ring* r, uint32_t layer, uint64_t clock) {
  const uint32_t slot = gh_ring_slot_index(r, clock);
  const size_t gi = (size_t)layer * r->total_slots + slot;
  r->clocks[gi] = clock;
  r->active[gi] = 1;
  if (layer == 0 && clock >= r->total_ingested) r->total_ingested = clock + 1;
  return slot;
}

// clearRecall (ring_buffer.zig:82-88)
void gh_ring_clear_recall(gh_ring* r) {
  for (size_t l = 0; l < r->num_layers; l++)
    memset(&r->active[l * r->total_slots + r->recall_start()], 0, r->num_recall);
}

// writeRecallKV's bookkeeping (ring_buffer.zig:90-99): recall slot `rank`
// becomes active with the stored memory's clock; returns its slot number.
uint32_t gh_ring_activate_recall(gh_ring* r, uint32_t layer, uint32_t rank, uint64_t clock) {
  const size_t slot = r->recall_start() + rank;
  const size_t gi = (size_t)layer * r->total_slots + slot;
  r->clocks[gi] = clock;
  r->active[gi] = 1;
  return (uint32_t)slot;
}

// getActiveSlots (ring_buffer.zig:101-136): anchors < min(clock + 1, A), then
// live window slots in slot order, then recall slots with clock <= now.
uint32_t gh_ring_active_slots(const gh_ring* r, uint32_t layer, uint64_t clock, uint32_t* out,
                              uint32_t cap) {
  const size_t base = (size_t)layer * r->total_slots;
  uint32_t n = 0;
  auto push = [&](size_t s) {
    if (n < cap) out[n] = (uint32_t)s;
    n++;
  };
  const size_t alim = clock + 1 < r->num_anchors ? (size_t)clock + 1 : r->num_anchors;
  for (size_t s = 0; s < alim; s++)
    if (r->active[base + s]) push(s);
  if (clock >= r->num_anchors) {
    const uint64_t minc = clock >= r->window_size ? clock - r->window_size + 1 : r->num_anchors;
    for (size_t s = r->num_anchors; s < r->recall_start(); s++) {
      if (!r->active[base + s]) continue;
      const uint64_t c = r->clocks[base + s];
      if (c >= minc && c <= clock) push(s);
    }
  }
  for (size_t s = r->recall_start(); s < r->total_slots; s++) {
    if (!r->active[base + s]) continue;
    if (r->clocks[base + s] <= clock) push(s);
  }
  return n;
}

}  // extern "C"

namespace gh {

gh_ring* ring_clone(const gh_ring* r) { return r ? new gh_ring(*r) : nullptr; }

// Layer `layer`'s clocks (as u32) and active flags of the first n slots; slots
// beyond the ring read as inactive.
void ring_state(const gh_ring* r, uint32_t layer, uint32_t* clocks, uint32_t* flags, uint32_t n) {
  const size_t base = (size_t)layer * r->total_slots;
  for (uint32_t s = 0; s < n; s++) {
    const bool in = s < r->total_slots;
    clocks[s] = in ? (uint32_t)r->clocks[base + s] : 0u;
    flags[s] = in ? r->active[base + s] : 0u;
  }
}

}  // namespace gh
