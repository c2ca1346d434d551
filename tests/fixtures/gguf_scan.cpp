/*
 * Runs libr9vx's GGUF reader (r9v_amd/csrc/gguf.hip, host code) over a
 * corpus file of records (u64 little-endian length, then that many bytes):
 * each record is parsed as a whole file and as a metadata-only table, and
 * an accepted file has every accessor walked (key-value items, tensor rows,
 * checked tensor ranges, entry hashes, matmul keys, a one-shard set).  One
 * output line per record: "<parse rc> <problem kinds> <table rc>".  Built
 * with AddressSanitizer / UndefinedBehaviorSanitizer by
 * tests/test_gguf_sanitize.py, so any out-of-bounds access or undefined
 * operation on hostile bytes ends the run with a report.
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "r9vx_gguf.h"

void r9vx_set_last_error(const std::string &) {}

static volatile uint64_t g_sink;

static void walk(const r9vx_gguf *f, const uint8_t *p, uint64_t n) {
    uint64_t ranges[6];
    r9vx_gguf_ranges(f, ranges);
    g_sink += r9vx_gguf_version(f) + r9vx_gguf_alignment(f) + r9vx_gguf_data_start(f) + r9vx_gguf_file_size(f) +
              ranges[5] + (uint64_t)r9vx_gguf_is_native(f);
    for (uint64_t i = 0; i < r9vx_gguf_n_kv(f); ++i) {
        const char *key = nullptr;
        uint64_t key_len = 0, count = 0;
        uint32_t type = 0, elem = 0;
        if (r9vx_gguf_kv_info(f, i, &key, &key_len, &type, &elem, &count) != 0) continue;
        for (uint64_t j = 0; j < key_len; ++j) g_sink += (uint8_t)key[j];
        if (key_len == strlen(key)) g_sink += (uint64_t)r9vx_gguf_find_kv(f, key);
        for (uint64_t item = 0; item < count; ++item) {
            r9vx_gguf_value v;
            if (r9vx_gguf_kv_value(f, i, item, &v) != 0) continue;
            g_sink += v.bits + v.type;
            for (uint64_t j = 0; v.str && j < v.str_len; ++j) g_sink += (uint8_t)v.str[j];
        }
    }
    for (uint64_t i = 0; i < r9vx_gguf_n_tensors(f); ++i) {
        r9vx_gguf_tensor t;
        if (r9vx_gguf_tensor_at(f, i, &t) != 0) continue;
        for (uint32_t d = 0; d < t.n_dims; ++d) g_sink += t.dims[d];
        g_sink += t.offset + t.nbytes + t.type + t.block_len + t.block_bytes;
        if (t.name_len != strlen(t.name)) continue; /* reachable by index only */
        g_sink += (uint64_t)r9vx_gguf_find_tensor(f, t.name);
        const uint8_t *data = nullptr;
        uint64_t nbytes = 0, hash = 0;
        if (r9vx_gguf_tensor_bytes(f, t.name, p, n, &data, &nbytes) == 0)
            for (uint64_t j = 0; j < nbytes; j += 4096) g_sink += data[j];
        if (r9vx_gguf_entry_xxh3(f, t.name, p, n, &hash) == 0) g_sink += hash;
        r9vx_matmul_static st;
        memset(&st, 0, sizeof st);
        g_sink += (uint64_t)r9vx_gguf_matmul_static(f, t.name, &st) + st.n + st.k;
    }
    r9vx_gguf_shards *s = nullptr;
    if (r9vx_gguf_shards_open(&f, 1, &s) == 0) {
        for (uint64_t i = 0; i < r9vx_gguf_shards_len(s); ++i) {
            uint32_t shard = 0;
            r9vx_gguf_tensor t;
            if (r9vx_gguf_shards_tensor_at(s, i, &shard, &t) == 0) g_sink += shard + t.nbytes;
        }
        r9vx_gguf_shards_free(s);
    }
}

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: gguf_scan CORPUS\n");
        return 2;
    }
    FILE *fp = fopen(argv[1], "rb");
    if (!fp) return 2;
    std::vector<uint8_t> all;
    uint8_t buf[65536];
    size_t got;
    while ((got = fread(buf, 1, sizeof buf, fp)) > 0) all.insert(all.end(), buf, buf + got);
    fclose(fp);
    size_t at = 0;
    while (at + 8 <= all.size()) {
        uint64_t len = 0;
        memcpy(&len, all.data() + at, 8);
        at += 8;
        if (len > all.size() - at) return 3;
        /* an exact-size heap copy, so that a read past the input is caught */
        std::vector<uint8_t> rec(all.begin() + (long)at, all.begin() + (long)(at + len));
        at += len;
        const uint8_t *p = rec.empty() ? nullptr : rec.data();
        r9vx_gguf *f = nullptr;
        const int rc = r9vx_gguf_parse(p, len, &f);
        const uint32_t kinds = r9vx_gguf_last_problems();
        if (rc == 0) {
            walk(f, p, len);
            r9vx_gguf_free(f);
        }
        r9vx_gguf *g = nullptr;
        const int rc2 = r9vx_gguf_parse_table(p, len, len, &g);
        if (rc2 == 0) {
            walk(g, p, len);
            r9vx_gguf_free(g);
        }
        printf("%d %u %d\n", rc, kinds, rc2);
    }
    return 0;
}
