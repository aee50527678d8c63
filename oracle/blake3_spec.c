/*
 * BLAKE3 hash (unkeyed mode, 32-byte output), written from the public BLAKE3
 * specification (O'Connor, Aumasson, Neves, Wilcox-O'Hearn, 2020, sections
 * 2.1-2.6).  TEST INFRASTRUCTURE ONLY: used by the oracle to reproduce the
 * reference's BLAKE3 digests of little-endian f32 outputs
 * (crates/pvlc-cpu-ref/tests/decoder_gqa_contract.rs:10, :103-109 and
 * crates/pvlc-cpu-ref/tests/decoder_decode_contract.rs:17-18, :520-543).
 *
 * The reference uses the `blake3` crate; that crate is not present in this
 * environment, so this file restates the published algorithm.  It is pinned by
 * the specification's published test vectors and by the model-lock digests of
 * the two configuration files the reference snapshot carries (tests/).
 */
#include <stdint.h>
#include <string.h>

#include "pvlc_oracle.h"

enum {
    CHUNK_START = 1u << 0,
    CHUNK_END = 1u << 1,
    PARENT = 1u << 2,
    ROOT = 1u << 3,
};

#define BLOCK_LEN 64u
#define CHUNK_LEN 1024u

static const uint32_t IV[8] = {
    0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
    0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u,
};

static const unsigned MSG_PERMUTATION[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};

static uint32_t rotr32(uint32_t w, unsigned c) { return (w >> c) | (w << (32u - c)); }

static void g(uint32_t s[16], unsigned a, unsigned b, unsigned c, unsigned d, uint32_t mx, uint32_t my) {
    s[a] = s[a] + s[b] + mx;
    s[d] = rotr32(s[d] ^ s[a], 16);
    s[c] = s[c] + s[d];
    s[b] = rotr32(s[b] ^ s[c], 12);
    s[a] = s[a] + s[b] + my;
    s[d] = rotr32(s[d] ^ s[a], 8);
    s[c] = s[c] + s[d];
    s[b] = rotr32(s[b] ^ s[c], 7);
}

static void round_fn(uint32_t s[16], const uint32_t m[16]) {
    g(s, 0, 4, 8, 12, m[0], m[1]);
    g(s, 1, 5, 9, 13, m[2], m[3]);
    g(s, 2, 6, 10, 14, m[4], m[5]);
    g(s, 3, 7, 11, 15, m[6], m[7]);
    g(s, 0, 5, 10, 15, m[8], m[9]);
    g(s, 1, 6, 11, 12, m[10], m[11]);
    g(s, 2, 7, 8, 13, m[12], m[13]);
    g(s, 3, 4, 9, 14, m[14], m[15]);
}

static void compress(const uint32_t cv[8], const uint32_t block[16], uint64_t counter, uint32_t block_len,
                     uint32_t flags, uint32_t out[16]) {
    uint32_t s[16] = {
        cv[0], cv[1], cv[2], cv[3], cv[4], cv[5], cv[6], cv[7],
        IV[0], IV[1], IV[2], IV[3],
        (uint32_t)counter, (uint32_t)(counter >> 32), block_len, flags,
    };
    uint32_t m[16];
    memcpy(m, block, sizeof(m));
    for (int r = 0; r < 7; ++r) {
        round_fn(s, m);
        if (r < 6) {
            uint32_t p[16];
            for (int i = 0; i < 16; ++i) p[i] = m[MSG_PERMUTATION[i]];
            memcpy(m, p, sizeof(m));
        }
    }
    for (int i = 0; i < 8; ++i) {
        s[i] ^= s[i + 8];
        s[i + 8] ^= cv[i];
    }
    memcpy(out, s, sizeof(s));
}

static void words_from_le_bytes(const uint8_t *bytes, size_t n_bytes, uint32_t words[16]) {
    uint8_t padded[BLOCK_LEN];
    memset(padded, 0, sizeof(padded));
    memcpy(padded, bytes, n_bytes);
    for (int i = 0; i < 16; ++i) {
        words[i] = (uint32_t)padded[4 * i] | ((uint32_t)padded[4 * i + 1] << 8) |
                   ((uint32_t)padded[4 * i + 2] << 16) | ((uint32_t)padded[4 * i + 3] << 24);
    }
}

/* A node whose compression is deferred until we know whether it is the root. */
typedef struct {
    uint32_t cv[8];
    uint32_t block[16];
    uint64_t counter;
    uint32_t block_len;
    uint32_t flags;
} output_t;

static void output_cv(const output_t *o, uint32_t cv_out[8]) {
    uint32_t full[16];
    compress(o->cv, o->block, o->counter, o->block_len, o->flags, full);
    memcpy(cv_out, full, 32);
}

static output_t parent_output(const uint32_t left[8], const uint32_t right[8]) {
    output_t o;
    memcpy(o.cv, IV, sizeof(IV));
    memcpy(o.block, left, 32);
    memcpy(o.block + 8, right, 32);
    o.counter = 0;
    o.block_len = BLOCK_LEN;
    o.flags = PARENT;
    return o;
}

/* Output of one chunk (<= 1024 bytes, at least one block even if empty). */
static output_t chunk_output(const uint8_t *chunk, size_t len, uint64_t chunk_counter) {
    uint32_t cv[8];
    memcpy(cv, IV, sizeof(IV));
    size_t n_blocks = len == 0 ? 1 : (len + BLOCK_LEN - 1) / BLOCK_LEN;
    for (size_t b = 0; b + 1 < n_blocks; ++b) {
        uint32_t words[16], full[16];
        words_from_le_bytes(chunk + b * BLOCK_LEN, BLOCK_LEN, words);
        uint32_t flags = b == 0 ? CHUNK_START : 0u;
        compress(cv, words, chunk_counter, BLOCK_LEN, flags, full);
        memcpy(cv, full, 32);
    }
    size_t last_off = (n_blocks - 1) * BLOCK_LEN;
    size_t last_len = len - last_off;
    output_t o;
    memcpy(o.cv, cv, sizeof(cv));
    words_from_le_bytes(chunk + last_off, last_len, o.block);
    o.counter = chunk_counter;
    o.block_len = (uint32_t)last_len;
    o.flags = CHUNK_END | (n_blocks == 1 ? CHUNK_START : 0u);
    return o;
}

void oracle_blake3(const uint8_t *input, size_t len, uint8_t out[32]) {
    /* Chaining-value stack of completed subtrees (spec section 5.1.2). */
    uint32_t stack[64][8];
    size_t depth = 0;
    uint64_t chunk_index = 0;
    size_t offset = 0;
    /* Every chunk except the last is final and merges into the stack. */
    while (len - offset > CHUNK_LEN) {
        output_t o = chunk_output(input + offset, CHUNK_LEN, chunk_index);
        uint32_t cv[8];
        output_cv(&o, cv);
        uint64_t total = chunk_index + 1;
        while ((total & 1u) == 0) {
            output_t p = parent_output(stack[depth - 1], cv);
            output_cv(&p, cv);
            --depth;
            total >>= 1;
        }
        memcpy(stack[depth++], cv, 32);
        offset += CHUNK_LEN;
        ++chunk_index;
    }
    output_t node = chunk_output(input + offset, len - offset, chunk_index);
    while (depth > 0) {
        uint32_t cv[8];
        output_cv(&node, cv);
        node = parent_output(stack[depth - 1], cv);
        --depth;
    }
    uint32_t full[16];
    compress(node.cv, node.block, node.counter, node.block_len, node.flags | ROOT, full);
    for (int i = 0; i < 8; ++i) {
        out[4 * i] = (uint8_t)full[i];
        out[4 * i + 1] = (uint8_t)(full[i] >> 8);
        out[4 * i + 2] = (uint8_t)(full[i] >> 16);
        out[4 * i + 3] = (uint8_t)(full[i] >> 24);
    }
}
