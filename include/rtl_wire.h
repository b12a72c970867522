/*
 * rtl_wire.h - the descriptor and completion contract between the 64-byte
 * software descriptor (hw_desc_t) and the RTL queue ports.
 *
 * The RTL model (rtl/desc_pkg.sv:8-27) carries a 192-bit packed desc_t and a
 * 56-bit packed completion_t. A SystemVerilog packed struct puts its first
 * declared field in the most significant bits; the 32-bit word images here
 * hold bits [32i + 31 : 32i] in word i, the layout the reference's simulator
 * bridge drives (verilator/rtl_bridge.cpp:114-146).
 *
 *   desc_t, MSB first:       opcode 8 | flags 8 | rollout_id 16 |
 *                            kv_arena_id 16 | prefix_id 16 | kv_offset 32 |
 *                            delta_offset 32 | seq_len 16 | max_tokens 16 |
 *                            reward_model_id 16 | reserved 16
 *   completion_t, MSB first: rollout_id 16 | status 8 | final_seq_len 16 |
 *                            reward_id 16
 *
 * One opcode and status namespace (the gap listed in
 * docs/descriptor_contract.md:188-200): DECODE 1, REWARD 2 and STOP 255 exist
 * on both sides; PREFILL 3 has no RTL value and the RTL's NOP 0 no software
 * value, so neither crosses. Completion status: DONE 1 (DESC_FLAG_DONE),
 * REWARD_NEEDED 2 (DESC_FLAG_NEEDS_REWARD), STOPPED 255.
 *
 * What does not cross: user_data and checksum_or_cookie (software metadata,
 * zero after an unpack), and any value wider than its RTL field - those make
 * the pack fail rather than truncate (the range checks of
 * verilator/rtl_bridge.cpp:171-172, made total).
 */
#pragma once

#include <stdint.h>
#include "hw_desc.h"
#include "rl_abi.h"

#define RTL_DESC_WORDS 6u /* 192 bits */
#define RTL_COMP_WORDS 2u /* 56 bits in two words, bits 56..63 zero */

#define RTL_DESC_OP_NOP 0u

#define RTL_COMP_STATUS_DONE          0x01u
#define RTL_COMP_STATUS_REWARD_NEEDED 0x02u
#define RTL_COMP_STATUS_STOPPED       0xFFu

RL_EXTERN_C_BEGIN

/* hw_desc_t -> desc_t words. 0, or -1 with nothing written when d or w is
 * NULL, the opcode has no RTL value, or a field exceeds its RTL width
 * (flags 8 bits; ids, lengths and reserved0 16 bits; offsets 32 bits). */
int rtl_desc_pack(const hw_desc_t *d, uint32_t w[RTL_DESC_WORDS]);

/* desc_t words -> hw_desc_t: every carried field zero-extended, user_data
 * and checksum_or_cookie zero. 0, or -1 with nothing written when a pointer
 * is NULL or the opcode has no software value (NOP, or not one of 1, 2, 255). */
int rtl_desc_unpack(const uint32_t w[RTL_DESC_WORDS], hw_desc_t *d);

/* The completion of a descriptor the worker returned -> completion_t words:
 * status DONE if DESC_FLAG_DONE is set, else REWARD_NEEDED if
 * DESC_FLAG_NEEDS_REWARD is set, else STOPPED for a STOP descriptor;
 * final_seq_len = seq_len, reward_id = reward_model_id. 0, or -1 with nothing
 * written when a pointer is NULL, no status applies (a decode descriptor the
 * worker returned with neither flag: it arrived with seq_len >= max_tokens,
 * which the RTL reports as DONE and the C worker leaves unmarked), or a field
 * exceeds 16 bits. */
int rtl_comp_pack(const hw_desc_t *done, uint32_t w[RTL_COMP_WORDS]);

/* completion_t words -> fields. 0, or -1 when a pointer is NULL, bits 56..63
 * are set, or the status is not one of 1, 2, 255. */
int rtl_comp_unpack(const uint32_t w[RTL_COMP_WORDS], uint32_t *rollout_id, uint32_t *status,
                    uint32_t *final_seq_len, uint32_t *reward_id);

RL_EXTERN_C_END
