/*
 * attention_decode.c - host half of the decode-attention ABI
 * (reference cu/attention_decode.cu:48-58 and :196-203).
 */
#include "attention_decode.h"

DecodeMicrokernelConfig
attention_decode_config_fixed128(void)
{
    DecodeMicrokernelConfig c;
    c.head_dim = DECODE_FIXED_HEAD_DIM;
    c.tokens_per_block = KV_LAYOUT_TOKENS_PER_BLOCK;
    c.tile_tokens = DECODE_TILE_TOKENS;
    c.prefetch_stages = DECODE_PREFETCH_STAGES;
    c.shared_bytes = DECODE_PREFETCH_STAGES * KV_LAYOUT_BLOCK_BYTES;
    return c;
}

DecodeStepResult
attention_decode_result_fixed128(uint32_t seq_len)
{
    uint32_t s = seq_len == 0u ? 1u : seq_len;
    if (s > KV_LAYOUT_TOKENS_PER_BLOCK)
        s = KV_LAYOUT_TOKENS_PER_BLOCK;
    DecodeStepResult r;
    r.path_kind = DECODE_PATH_FIXED128;
    r.token_id = 0;
    r.bytes_touched = s * DECODE_FIXED_HEAD_DIM * KV_LAYOUT_SCALAR_BYTES * 2u;
    r.tile_count = (s + DECODE_TILE_TOKENS - 1u) / DECODE_TILE_TOKENS;
    r.cycle_estimate = (uint64_t)r.tile_count * (uint64_t)DECODE_FIXED_HEAD_DIM * 24ull;
    return r;
}
