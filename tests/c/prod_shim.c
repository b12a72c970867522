/* Exports the runtime's header-inline ring functions (include/*.h) so tests can
 * drive them with the same traces as the oracle and the reference build. */
#include "completion.h"
#include "hw_ring.h"
#include "kv_layout.h"
#include "request.h"
#include "ring.h"

int prod_hw_ring_push(hw_ring_t *r, const hw_desc_t *d) { return hw_ring_push(r, d); }
int prod_hw_ring_pop(hw_ring_t *r, hw_desc_t *d) { return hw_ring_pop(r, d); }
int prod_hw_ring_full(hw_ring_t *r) { return hw_ring_full(r); }
int prod_hw_ring_empty(hw_ring_t *r) { return hw_ring_empty(r); }
uint32_t prod_ring_acquire(CommandRing *r, uint32_t n) { return ring_acquire(r, n); }
void prod_ring_commit(CommandRing *r, uint32_t n) { ring_commit(r, n); }
int prod_ring_consume(CommandRing *r, Descriptor *d) { return ring_consume(r, d); }
int prod_comp_ring_push(CompletionRing *r, const Completion *c) { return comp_ring_push(r, c); }
int prod_comp_ring_poll(CompletionRing *r, Completion *c) { return comp_ring_poll(r, c); }
uint32_t prod_req_ring_acquire(RequestRing *r) { return req_ring_acquire(r); }
void prod_req_ring_commit(RequestRing *r) { req_ring_commit(r); }
int prod_req_ring_consume(RequestRing *r, RolloutRequest *o) { return req_ring_consume(r, o); }
int prod_done_ring_push(DoneRing *r, const RolloutDone *d) { return done_ring_push(r, d); }
int prod_done_ring_pop(DoneRing *r, RolloutDone *o) { return done_ring_pop(r, o); }
void prod_kv_layout_desc_fixed128(KvLayoutDesc *out) { *out = kv_layout_desc_fixed128(); }
uint32_t prod_kv_layout_block_offset_bytes(uint32_t i) { return kv_layout_block_offset_bytes(i); }
uint32_t prod_kv_layout_k_offset_bytes(uint32_t t) { return kv_layout_k_offset_bytes(t); }
uint32_t prod_kv_layout_v_offset_bytes(uint32_t t) { return kv_layout_v_offset_bytes(t); }
