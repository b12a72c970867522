/*
 * rtl_wire.c - hw_desc_t <-> RTL desc_t / completion_t word images
 * (rtl/desc_pkg.sv:8-27; word layout of verilator/rtl_bridge.cpp:114-146).
 */
#include "rtl_wire.h"

#include <string.h>

static int
opcode_crosses(uint32_t op)
{
    return op == DESC_OP_DECODE || op == DESC_OP_REWARD || op == DESC_OP_STOP;
}

int
rtl_desc_pack(const hw_desc_t *d, uint32_t w[RTL_DESC_WORDS])
{
    if (!d || !w || !opcode_crosses(d->opcode))
        return -1;
    if (d->flags > 0xFFu || d->rollout_id > 0xFFFFu || d->kv_arena_id > 0xFFFFu || d->prefix_id > 0xFFFFu ||
        d->seq_len > 0xFFFFu || d->max_tokens > 0xFFFFu || d->reward_model_id > 0xFFFFu || d->reserved0 > 0xFFFFu ||
        d->kv_offset > 0xFFFFFFFFull || d->delta_offset > 0xFFFFFFFFull)
        return -1;
    /* bits 191..0, most significant field first */
    w[5] = ((uint32_t)d->opcode << 24) | ((uint32_t)d->flags << 16) | d->rollout_id;
    w[4] = (d->kv_arena_id << 16) | d->prefix_id;
    w[3] = (uint32_t)d->kv_offset;
    w[2] = (uint32_t)d->delta_offset;
    w[1] = (d->seq_len << 16) | d->max_tokens;
    w[0] = (d->reward_model_id << 16) | d->reserved0;
    return 0;
}

int
rtl_desc_unpack(const uint32_t w[RTL_DESC_WORDS], hw_desc_t *d)
{
    if (!w || !d)
        return -1;
    const uint32_t op = w[5] >> 24;
    if (!opcode_crosses(op))
        return -1;
    memset(d, 0, sizeof(*d));
    d->opcode = (uint16_t)op;
    d->flags = (uint16_t)((w[5] >> 16) & 0xFFu);
    d->rollout_id = w[5] & 0xFFFFu;
    d->kv_arena_id = w[4] >> 16;
    d->prefix_id = w[4] & 0xFFFFu;
    d->kv_offset = w[3];
    d->delta_offset = w[2];
    d->seq_len = w[1] >> 16;
    d->max_tokens = w[1] & 0xFFFFu;
    d->reward_model_id = w[0] >> 16;
    d->reserved0 = w[0] & 0xFFFFu;
    return 0;
}

int
rtl_comp_pack(const hw_desc_t *done, uint32_t w[RTL_COMP_WORDS])
{
    if (!done || !w)
        return -1;
    uint32_t status;
    if (done->opcode == DESC_OP_STOP)
        status = RTL_COMP_STATUS_STOPPED;
    else if (done->flags & DESC_FLAG_DONE)
        status = RTL_COMP_STATUS_DONE;
    else if (done->flags & DESC_FLAG_NEEDS_REWARD)
        status = RTL_COMP_STATUS_REWARD_NEEDED;
    else
        return -1;
    if (done->rollout_id > 0xFFFFu || done->seq_len > 0xFFFFu || done->reward_model_id > 0xFFFFu)
        return -1;
    /* bits 55..0: rollout_id 55..40, status 39..32, final_seq_len 31..16, reward_id 15..0 */
    w[1] = (done->rollout_id << 8) | status;
    w[0] = (done->seq_len << 16) | done->reward_model_id;
    return 0;
}

int
rtl_comp_unpack(const uint32_t w[RTL_COMP_WORDS], uint32_t *rollout_id, uint32_t *status, uint32_t *final_seq_len,
                uint32_t *reward_id)
{
    if (!w || !rollout_id || !status || !final_seq_len || !reward_id || (w[1] >> 24) != 0)
        return -1;
    const uint32_t st = w[1] & 0xFFu;
    if (st != RTL_COMP_STATUS_DONE && st != RTL_COMP_STATUS_REWARD_NEEDED && st != RTL_COMP_STATUS_STOPPED)
        return -1;
    *rollout_id = (w[1] >> 8) & 0xFFFFu;
    *status = st;
    *final_seq_len = w[0] >> 16;
    *reward_id = w[0] & 0xFFFFu;
    return 0;
}
