/*
 * r9vx_xxh3.h -- XXH3-64 (seed 0, default secret) for the per-entry tensor
 * checksum of GGUF ingestion.  Host code.
 *
 * R9V hashes every tensor entry with xxh3_64 (crates/r9v-common/src/hash.rs:12,
 * called by GgufFile::entry_xxh3, crates/r9v-format/src/container.rs:2136);
 * that function is the xxhash-rust crate's XXH3 with seed 0.  This is an own
 * scalar implementation of the published XXH3 algorithm (xxHash 0.8 format,
 * Yann Collet, BSD-2): length classes 0, 1-3, 4-8, 9-16, 17-128, 129-240 and the
 * striped long form (64-byte stripes, 16 stripes per 1 KiB block, accumulator
 * scramble per block).  The 192-byte default secret and the prime constants
 * are the algorithm's published constants.  Little-endian reads only (x86-64).
 */
#pragma once

#include <stdint.h>
#include <string.h>

namespace r9vx_xxh3 {

constexpr uint64_t P32_1 = 0x9E3779B1u, P32_2 = 0x85EBCA77u, P32_3 = 0xC2B2AE3Du;
constexpr uint64_t P64_1 = 0x9E3779B185EBCA87ull, P64_2 = 0xC2B2AE3D27D4EB4Full,
                   P64_3 = 0x165667B19E3779F9ull, P64_4 = 0x85EBCA77C2B2AE63ull,
                   P64_5 = 0x27D4EB2F165667C5ull;
constexpr uint64_t PMX_1 = 0x165667919E3779F9ull, PMX_2 = 0x9FB21C651E98DF25ull;

constexpr int kSecretSize = 192;
alignas(64) static const uint8_t kSecret[kSecretSize] = {
    0xb8, 0xfe, 0x6c, 0x39, 0x23, 0xa4, 0x4b, 0xbe, 0x7c, 0x01, 0x81, 0x2c, 0xf7, 0x21, 0xad, 0x1c,
    0xde, 0xd4, 0x6d, 0xe9, 0x83, 0x90, 0x97, 0xdb, 0x72, 0x40, 0xa4, 0xa4, 0xb7, 0xb3, 0x67, 0x1f,
    0xcb, 0x79, 0xe6, 0x4e, 0xcc, 0xc0, 0xe5, 0x78, 0x82, 0x5a, 0xd0, 0x7d, 0xcc, 0xff, 0x72, 0x21,
    0xb8, 0x08, 0x46, 0x74, 0xf7, 0x43, 0x24, 0x8e, 0xe0, 0x35, 0x90, 0xe6, 0x81, 0x3a, 0x26, 0x4c,
    0x3c, 0x28, 0x52, 0xbb, 0x91, 0xc3, 0x00, 0xcb, 0x88, 0xd0, 0x65, 0x8b, 0x1b, 0x53, 0x2e, 0xa3,
    0x71, 0x64, 0x48, 0x97, 0xa2, 0x0d, 0xf9, 0x4e, 0x38, 0x19, 0xef, 0x46, 0xa9, 0xde, 0xac, 0xd8,
    0xa8, 0xfa, 0x76, 0x3f, 0xe3, 0x9c, 0x34, 0x3f, 0xf9, 0xdc, 0xbb, 0xc7, 0xc7, 0x0b, 0x4f, 0x1d,
    0x8a, 0x51, 0xe0, 0x4b, 0xcd, 0xb4, 0x59, 0x31, 0xc8, 0x9f, 0x7e, 0xc9, 0xd9, 0x78, 0x73, 0x64,
    0xea, 0xc5, 0xac, 0x83, 0x34, 0xd3, 0xeb, 0xc3, 0xc5, 0x81, 0xa0, 0xff, 0xfa, 0x13, 0x63, 0xeb,
    0x17, 0x0d, 0xdd, 0x51, 0xb7, 0xf0, 0xda, 0x49, 0xd3, 0x16, 0x55, 0x26, 0x29, 0xd4, 0x68, 0x9e,
    0x2b, 0x16, 0xbe, 0x58, 0x7d, 0x47, 0xa1, 0xfc, 0x8f, 0xf8, 0xb8, 0xd1, 0x7a, 0xd0, 0x31, 0xce,
    0x45, 0xcb, 0x3a, 0x8f, 0x95, 0x16, 0x04, 0x28, 0xaf, 0xd7, 0xfb, 0xca, 0xbb, 0x4b, 0x40, 0x7e,
};

inline uint64_t rd64(const uint8_t *p) { uint64_t v; memcpy(&v, p, 8); return v; }
inline uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
inline uint64_t rotl(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }
inline uint64_t bswap64(uint64_t v) { return __builtin_bswap64(v); }
inline uint32_t bswap32(uint32_t v) { return __builtin_bswap32(v); }

/* Low 64 bits XOR high 64 bits of the 128-bit product. */
inline uint64_t fold_mul(uint64_t a, uint64_t b) {
    const unsigned __int128 p = (unsigned __int128)a * b;
    return (uint64_t)p ^ (uint64_t)(p >> 64);
}

inline uint64_t avalanche_xxh64(uint64_t h) {
    h ^= h >> 33;
    h *= P64_2;
    h ^= h >> 29;
    h *= P64_3;
    h ^= h >> 32;
    return h;
}

inline uint64_t avalanche(uint64_t h) {
    h ^= h >> 37;
    h *= PMX_1;
    h ^= h >> 32;
    return h;
}

inline uint64_t rrmxmx(uint64_t h, uint64_t len) {
    h ^= rotl(h, 49) ^ rotl(h, 24);
    h *= PMX_2;
    h ^= (h >> 35) + len;
    h *= PMX_2;
    h ^= h >> 28;
    return h;
}

/* 16 input bytes against 16 secret bytes (seed 0). */
inline uint64_t mix16(const uint8_t *in, const uint8_t *sec) {
    return fold_mul(rd64(in) ^ rd64(sec), rd64(in + 8) ^ rd64(sec + 8));
}

inline uint64_t hash_0to16(const uint8_t *in, uint64_t len) {
    if (len > 8) {
        const uint64_t lo = rd64(in) ^ (rd64(kSecret + 24) ^ rd64(kSecret + 32));
        const uint64_t hi = rd64(in + len - 8) ^ (rd64(kSecret + 40) ^ rd64(kSecret + 48));
        return avalanche(len + bswap64(lo) + hi + fold_mul(lo, hi));
    }
    if (len >= 4) {
        const uint64_t both = (uint64_t)rd32(in + len - 4) + ((uint64_t)rd32(in) << 32);
        return rrmxmx(both ^ (rd64(kSecret + 8) ^ rd64(kSecret + 16)), len);
    }
    if (len > 0) {
        const uint32_t packed = ((uint32_t)in[0] << 16) | ((uint32_t)in[len >> 1] << 24) |
                                (uint32_t)in[len - 1] | ((uint32_t)len << 8);
        return avalanche_xxh64((uint64_t)(packed ^ (rd32(kSecret) ^ rd32(kSecret + 4))));
    }
    return avalanche_xxh64(rd64(kSecret + 56) ^ rd64(kSecret + 64));
}

inline uint64_t hash_17to128(const uint8_t *in, uint64_t len) {
    uint64_t acc = len * P64_1;
    /* pairs of 16-byte lanes from both ends, outermost pair on the first secret bytes */
    const uint64_t pairs = (len - 1) / 32;  /* 0..3 extra pairs beyond the first */
    for (uint64_t i = 0; i <= pairs; ++i) {
        acc += mix16(in + 16 * i, kSecret + 32 * i);
        acc += mix16(in + len - 16 * (i + 1), kSecret + 32 * i + 16);
    }
    return avalanche(acc);
}

inline uint64_t hash_129to240(const uint8_t *in, uint64_t len) {
    uint64_t acc = len * P64_1;
    for (int i = 0; i < 8; ++i) acc += mix16(in + 16 * i, kSecret + 16 * i);
    acc = avalanche(acc);
    const uint64_t rounds = len / 16;
    for (uint64_t i = 8; i < rounds; ++i) acc += mix16(in + 16 * i, kSecret + 16 * (i - 8) + 3);
    acc += mix16(in + len - 16, kSecret + 136 - 17);
    return avalanche(acc);
}

inline void accumulate_stripe(uint64_t acc[8], const uint8_t *in, const uint8_t *sec) {
    for (int i = 0; i < 8; ++i) {
        const uint64_t v = rd64(in + 8 * i);
        const uint64_t k = v ^ rd64(sec + 8 * i);
        acc[i ^ 1] += v;
        acc[i] += (k & 0xFFFFFFFFull) * (k >> 32);
    }
}

inline void scramble(uint64_t acc[8], const uint8_t *sec) {
    for (int i = 0; i < 8; ++i) {
        uint64_t a = acc[i];
        a ^= a >> 47;
        a ^= rd64(sec + 8 * i);
        a *= P32_1;
        acc[i] = a;
    }
}

inline uint64_t hash_long(const uint8_t *in, uint64_t len) {
    constexpr uint64_t kStripe = 64, kStripesPerBlock = (kSecretSize - kStripe) / 8;
    constexpr uint64_t kBlock = kStripe * kStripesPerBlock;
    uint64_t acc[8] = {P32_3, P64_1, P64_2, P64_3, P64_4, P32_2, P64_5, P32_1};
    const uint64_t blocks = (len - 1) / kBlock;
    for (uint64_t b = 0; b < blocks; ++b) {
        for (uint64_t s = 0; s < kStripesPerBlock; ++s)
            accumulate_stripe(acc, in + b * kBlock + s * kStripe, kSecret + s * 8);
        scramble(acc, kSecret + kSecretSize - kStripe);
    }
    const uint64_t tail_stripes = ((len - 1) - blocks * kBlock) / kStripe;
    for (uint64_t s = 0; s < tail_stripes; ++s)
        accumulate_stripe(acc, in + blocks * kBlock + s * kStripe, kSecret + s * 8);
    accumulate_stripe(acc, in + len - kStripe, kSecret + kSecretSize - kStripe - 7);
    uint64_t h = len * P64_1;
    for (int i = 0; i < 4; ++i)
        h += fold_mul(acc[2 * i] ^ rd64(kSecret + 11 + 16 * i), acc[2 * i + 1] ^ rd64(kSecret + 11 + 16 * i + 8));
    return avalanche(h);
}

inline uint64_t xxh3_64(const void *data, uint64_t len) {
    const uint8_t *in = static_cast<const uint8_t *>(data);
    if (len <= 16) return hash_0to16(in, len);
    if (len <= 128) return hash_17to128(in, len);
    if (len <= 240) return hash_129to240(in, len);
    return hash_long(in, len);
}

}  // namespace r9vx_xxh3
