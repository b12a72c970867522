/*
 * ref_shim.c - compiled only into oracle/_ref/libgbref.so, against the
 * reference headers. Re-exports the reference's header-inline ring and layout
 * functions (which have no symbols of their own) so tests can replay traces
 * through the reference code itself. No reference logic is restated here.
 */
#include "completion.h"
#include "hw_ring.h"
#include "kv_layout.h"
#include "request.h"
#include "ring.h"

int ref_hw_ring_push(hw_ring_t *r, const hw_desc_t *d) { return hw_ring_push(r, d); }
int ref_hw_ring_pop(hw_ring_t *r, hw_desc_t *d) { return hw_ring_pop(r, d); }
int ref_hw_ring_full(hw_ring_t *r) { return hw_ring_full(r); }
int ref_hw_ring_empty(hw_ring_t *r) { return hw_ring_empty(r); }

uint32_t ref_ring_acquire(CommandRing *r, uint32_t n) { return ring_acquire(r, n); }
void ref_ring_commit(CommandRing *r, uint32_t n) { ring_commit(r, n); }
int ref_ring_consume(CommandRing *r, Descriptor *d) { return ring_consume(r, d); }

int ref_comp_ring_push(CompletionRing *r, const Completion *c) { return comp_ring_push(r, c); }
int ref_comp_ring_poll(CompletionRing *r, Completion *c) { return comp_ring_poll(r, c); }

uint32_t ref_req_ring_acquire(RequestRing *r) { return req_ring_acquire(r); }
void ref_req_ring_commit(RequestRing *r) { req_ring_commit(r); }
int ref_req_ring_consume(RequestRing *r, RolloutRequest *o) { return req_ring_consume(r, o); }
int ref_done_ring_push(DoneRing *r, const RolloutDone *d) { return done_ring_push(r, d); }
int ref_done_ring_pop(DoneRing *r, RolloutDone *o) { return done_ring_pop(r, o); }

void ref_kv_layout_desc_fixed128(KvLayoutDesc *out) { *out = kv_layout_desc_fixed128(); }
uint32_t ref_kv_layout_block_offset_bytes(uint32_t i) { return kv_layout_block_offset_bytes(i); }
uint32_t ref_kv_layout_k_offset_bytes(uint32_t t) { return kv_layout_k_offset_bytes(t); }
uint32_t ref_kv_layout_v_offset_bytes(uint32_t t) { return kv_layout_v_offset_bytes(t); }
