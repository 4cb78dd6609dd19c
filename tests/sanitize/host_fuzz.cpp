// host_fuzz.cpp — host-side checks of libturboquant's C++ sources, built with
// AddressSanitizer + UndefinedBehaviorSanitizer (tests/test_sanitize.py).
//
//   host_fuzz abi                  C-ABI host paths: layouts, NULL -> -1,
//                                  invalid configs -> -2 with a message, the
//                                  page allocator and block table
//   host_fuzz fuzz SEED ITERS DIR  seeded mutation fuzz of the store readers
//                                  (.meta / fp16 .bin torch.save archives,
//                                  their pickles, .bin footers, manifest.json)
//   host_fuzz parse FILE...        reads each file as a .meta and as an fp16
//                                  .bin and prints the return codes
//
// A reader may accept or reject an input (rc 0 or -2); anything else, or a
// sanitizer report, ends the run with a non-zero status at the first failure.
#include <sys/stat.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "tq_turbo_prod_launch.h"
#include "turboquant.h"

namespace {

#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            std::fprintf(stderr, "CHECK failed %s:%d: %s (last error: %s)\n",     \
                         __FILE__, __LINE__, #cond, tq_last_error());            \
            std::exit(1);                                                        \
        }                                                                        \
    } while (0)

// splitmix64 (Steele, Lea, Flood 2014)
struct Rng {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    uint64_t below(uint64_t n) { return n ? next() % n : 0; }
};

std::string read_all(const std::string& p) {
    std::string s;
    if (FILE* f = std::fopen(p.c_str(), "rb")) {
        char buf[65536];
        size_t n;
        while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) s.append(buf, n);
        std::fclose(f);
    }
    return s;
}

void write_all(const std::string& p, const std::string& s) {
    FILE* f = std::fopen(p.c_str(), "wb");
    CHECK(f);
    CHECK(std::fwrite(s.data(), 1, s.size(), f) == s.size());
    std::fclose(f);
}

// ---------------------------------------------------------------------------
// abi
// ---------------------------------------------------------------------------
// The C++ launchers (include/tq_turbo_prod.cuh:45-101 semantics): results of
// the C entries, errors as std::runtime_error with the entry's message.
template <class F>
bool throws(F f, const char* needle) {
    try {
        f();
    } catch (const std::runtime_error& e) {
        return std::strstr(e.what(), needle) != nullptr;
    }
    return false;
}

void run_cxx_launchers(const TQConfig& cfg) {
    TQTurboProdPageLayout a{};
    CHECK(tq_make_turbo_prod_layout(&cfg, &a) == 0);
    const TQTurboProdPageLayout b = make_tq_turbo_prod_page_layout(cfg);
    CHECK(std::memcmp(&a, &b, sizeof a) == 0);
    TQConfig bad = cfg;  // the factory computes any shape (as the reference's)
    bad.head_dim = 3;
    const TQTurboProdPageLayout c = make_tq_turbo_prod_page_layout(bad);
    CHECK(tq_make_turbo_prod_layout(&bad, &a) == 0 && std::memcmp(&a, &c, sizeof a) == 0);
    CHECK(tq_make_turbo_prod_layout(&cfg, &a) == 0);
    // null pointers and a bad configuration fail before any launch
    CHECK(throws([&] { launch_tq_turbo_prod_pack_kv(nullptr, nullptr, nullptr, nullptr, a, cfg, 1,
                                                    nullptr); }, "NULL"));
    CHECK(throws([&] { launch_tq_turbo_prod_dequant_kv(nullptr, nullptr, nullptr, nullptr, a, cfg,
                                                       1, nullptr); }, "NULL"));
    CHECK(throws([&] { launch_tq_turbo_prod_fused_attention_logits(nullptr, nullptr, nullptr,
                                                                   nullptr, a, cfg, 1, 1,
                                                                   nullptr); }, "NULL"));
    CHECK(throws([&] { launch_tq_turbo_prod_fused_attention_output(nullptr, nullptr, nullptr,
                                                                   nullptr, a, cfg, 1, 1,
                                                                   nullptr); }, "NULL"));
    uint16_t h[4] = {};
    int32_t sl[1] = {0};
    uint8_t pg[4] = {};
    float dbg[4] = {};
    CHECK(throws([&] { launch_tq_turbo_prod_pack_kv(h, h, sl, pg, a, bad, 1, nullptr); },
                 "head_dim"));
    // a debug buffer routes the call to the debug pack (a stand-in here)
    CHECK(throws([&] { launch_tq_turbo_prod_pack_kv(h, h, sl, pg, a, cfg, 1, nullptr, dbg); },
                 "pack debug"));
}

int run_abi() {
    TQConfig cfg;
    CHECK(tq_make_default_config(&cfg) == 0);
    CHECK(tq_make_default_config(nullptr) == -1);
    run_cxx_launchers(cfg);
    // Layout factories over a grid of shapes (no device involved).
    for (int H : {1, 2, 3, 8, 64})
        for (int D : {2, 16, 64, 128, 256})
            for (int B : {1, 7, 16, 32}) {
                TQConfig c = cfg;
                c.num_kv_heads = H;
                c.head_dim = D;
                c.block_size = B;
                TQTurboProdPageLayout lp;
                TQTurbomsePageLayout lm;
                TQQJLPageLayout lq;
                TQDensePageLayout ld;
                CHECK(tq_make_turbo_prod_layout(&c, &lp) == 0);
                CHECK(tq_make_turbo_mse_layout(&c, &lm) == 0);
                CHECK(tq_make_qjl_layout(&c, &lq) == 0);
                CHECK(tq_make_dense_layout(&c, &ld) == 0);
                CHECK(lp.page_size_bytes >= (size_t)B * H * D);
                CHECK(lm.page_size_bytes >= (size_t)B * H * D);
            }
    TQTurboProdPageLayout lp;
    TQTurbomsePageLayout lm;
    CHECK(tq_make_turbo_prod_layout(&cfg, nullptr) == -1);
    CHECK(tq_make_turbo_mse_layout(nullptr, &lm) == -1);
    cfg.num_kv_heads = 2;
    CHECK(tq_make_turbo_prod_layout(&cfg, &lp) == 0);
    CHECK(tq_make_turbo_mse_layout(&cfg, &lm) == 0);

    // Fake device pointers: validation fails or the launch stand-in throws
    // before anything is dereferenced.
    uint16_t* fk = reinterpret_cast<uint16_t*>(0x1000);
    int32_t* fs = reinterpret_cast<int32_t*>(0x2000);
    uint8_t* fp = reinterpret_cast<uint8_t*>(0x3000);
    CHECK(tq_launch_turbo_prod_pack_kv(nullptr, fk, fs, fp, &lp, &cfg, 4, nullptr) == -1);
    CHECK(tq_launch_turbo_prod_dequant_kv(fp, fs, fk, nullptr, &lp, &cfg, 4, nullptr) == -1);
    CHECK(tq_launch_turbo_prod_pack_kv_debug(fk, fk, nullptr, fp, &lp, &cfg, 4, nullptr, nullptr,
                                             nullptr, nullptr, nullptr, nullptr, nullptr) == -1);
    CHECK(tq_launch_turbo_prod_fused_attention_output(fk, fp, fs, fk, nullptr, &cfg, 8, 4,
                                                      nullptr) == -1);
    CHECK(tq_launch_turbo_mse_pack_kv(fk, fk, fs, fp, &lm, nullptr, 4, nullptr) == -1);
    // Invalid configurations: rc -2 and a message.
    TQConfig bad = cfg;
    bad.head_dim = 256;
    CHECK(tq_launch_turbo_prod_pack_kv(fk, fk, fs, fp, &lp, &bad, 4, nullptr) == -2);
    CHECK(std::strstr(tq_last_error(), "head_dim > 128") != nullptr);
    bad.head_dim = 96;
    CHECK(tq_launch_turbo_mse_dequant_kv(fp, fs, fk, fk, &lm, &bad, 4, nullptr) == -2);
    bad = cfg;
    bad.num_kv_heads = 0;
    CHECK(tq_launch_turbo_prod_dequant_kv(fp, fs, fk, fk, &lp, &bad, 4, nullptr) == -2);
    CHECK(tq_launch_turbo_prod_pack_kv(fk, fk, fs, fp, &lp, &cfg, 0, nullptr) == -2);
    CHECK(tq_launch_turbo_prod_pack_kv(fk, fk, fs, fp, &lp, &cfg, 4, nullptr) == -2);
    CHECK(std::strstr(tq_last_error(), "sanitizer build") != nullptr);
    TQTurboProdPageLayout wrong = lp;
    wrong.k4_bytes_per_token_head = 7;
    CHECK(tq_launch_turbo_prod_pack_kv(fk, fk, fs, fp, &wrong, &cfg, 4, nullptr) == -2);
    // Multi-layer entries: host arrays of device pointers, checked per layer.
    const uint16_t* ks2[2] = {fk, fk};
    const uint16_t* vs2[2] = {fk, nullptr};
    uint8_t* ps2[2] = {fp, fp};
    const uint8_t* cps2[2] = {fp, fp};
    uint16_t* os2[2] = {fk, fk};
    CHECK(tq_launch_turbo_prod_pack_kv_layers(nullptr, ks2, fs, ps2, 2, &lp, &cfg, 4, nullptr) ==
          -1);
    CHECK(tq_launch_turbo_prod_pack_kv_layers(ks2, vs2, fs, ps2, 2, &lp, &cfg, 4, nullptr) == -2);
    CHECK(std::strstr(tq_last_error(), "null input or pool pointer") != nullptr);
    CHECK(tq_launch_turbo_mse_pack_kv_layers(ks2, ks2, fs, ps2, -1, &lm, &cfg, 4, nullptr) == -2);
    CHECK(tq_launch_turbo_prod_pack_kv_layers(ks2, ks2, fs, ps2, 2, &lp, &cfg, 0, nullptr) == -2);
    CHECK(tq_launch_turbo_prod_pack_kv_layers(ks2, ks2, fs, ps2, 2, &lp, &cfg, 4, nullptr) == -2);
    CHECK(std::strstr(tq_last_error(), "sanitizer build") != nullptr);
    CHECK(tq_launch_turbo_prod_dequant_kv_layers(cps2, fs, os2, nullptr, 2, &lp, &cfg, 4, 0,
                                                 nullptr) == -1);
    CHECK(tq_launch_turbo_mse_dequant_kv_layers(cps2, fs, os2, os2, 2, &lm, &cfg, 1 << 30, 0,
                                                nullptr) == -2);
    CHECK(tq_launch_turbo_prod_paged_attention(fk, fp, fs, 0, fs, fs, fk, &lp, &cfg, 8, 16,
                                               nullptr) == -2);
    CHECK(tq_launch_turbo_prod_paged_attention(fk, fp, fs, 1, fs, fs, fk, &lp, &cfg, 8, 17,
                                               nullptr) == -2);

    // Page allocator + block table (reference semantics: LIFO, pages 0, 1, 2
    // first, "out of blocks"); a caller-provided pool pointer, so no device.
    TQAllocator* a = nullptr;
    CHECK(tq_allocator_create(4288, 3, fp, &a) == 0);
    int32_t b0, b1, b2, b3;
    CHECK(tq_allocator_alloc_block(a, &b0) == 0 && b0 == 0);
    CHECK(tq_allocator_alloc_block(a, &b1) == 0 && b1 == 1);
    CHECK(tq_allocator_free_block(a, b0) == 0);
    CHECK(tq_allocator_alloc_block(a, &b2) == 0 && b2 == 0);
    CHECK(tq_allocator_alloc_block(a, &b3) == 0 && b3 == 2);
    int32_t none = 0;
    CHECK(tq_allocator_alloc_block(a, &none) == 0 && none == -1);
    for (int32_t b : {b1, b2, b3}) CHECK(tq_allocator_free_block(a, b) == 0);
    int nf = 0;
    CHECK(tq_allocator_num_free(a, &nf) == 0 && nf == 3);
    TQBlockTable* t = nullptr;
    CHECK(tq_block_table_create(a, 16, &t) == 0);
    std::vector<int32_t> slots(64);
    CHECK(tq_block_table_build_slot_map(t, 5, 20, slots.data()) == 0);
    {  // LIFO: the last page freed (2) comes out first, then 0
        int32_t bl[4];
        int n = 0;
        CHECK(tq_block_table_blocks(t, 5, bl, 4, &n) == 0 && n == 2 && bl[0] == 2 && bl[1] == 0);
        for (int i = 0; i < 20; ++i) CHECK(slots[i] == bl[i / 16] * 16 + i % 16);
    }
    CHECK(tq_block_table_build_slot_map(t, 6, 40, slots.data()) == -2);  // out of blocks
    CHECK(std::strstr(tq_last_error(), "out of blocks") != nullptr);
    int ntok = 0;
    CHECK(tq_block_table_num_tokens(t, 5, &ntok) == 0 && ntok == 20);
    ntok = -1;
    const int rc6 = tq_block_table_num_tokens(t, 6, &ntok);  // unchanged: absent or empty
    CHECK((rc6 == 0 && ntok == 0) || rc6 == -2);
    int32_t blocks[8];
    int nb = 0;
    CHECK(tq_block_table_blocks(t, 5, blocks, 8, &nb) == 0 && nb == 2);
    CHECK(tq_block_table_blocks(t, 5, blocks, 1, &nb) == 0 && nb == 2);  // capped copy
    CHECK(tq_block_table_free_sequence(t, 5) == 0);
    CHECK(tq_allocator_num_free(a, &nf) == 0 && nf == 3);
    CHECK(tq_block_table_destroy(t) == 0);
    CHECK(tq_allocator_destroy(a) == 0);
    std::printf("abi ok\n");
    return 0;
}

// ---------------------------------------------------------------------------
// fuzz
// ---------------------------------------------------------------------------
struct Rec {
    std::string name, data;
};

// The stored records of a zip, found by walking the local headers (enough
// for the archives written by this library, which are the seeds).
std::vector<Rec> local_records(const std::string& z) {
    std::vector<Rec> out;
    size_t p = 0;
    while (p + 30 <= z.size()) {
        uint32_t sig, size;
        uint16_t nl, xl;
        std::memcpy(&sig, z.data() + p, 4);
        if (sig != 0x04034b50u) break;
        std::memcpy(&size, z.data() + p + 18, 4);
        std::memcpy(&nl, z.data() + p + 26, 2);
        std::memcpy(&xl, z.data() + p + 28, 2);
        const size_t d = p + 30 + nl + xl;
        CHECK(d + size <= z.size());
        out.push_back({z.substr(p + 30, nl), z.substr(d, size)});
        p = d + size;
    }
    return out;
}

uint32_t crc32_bytes(const std::string& s) {
    uint32_t c = 0xFFFFFFFFu;
    for (unsigned char b : s) {
        c ^= b;
        for (int k = 0; k < 8; ++k) c = (c >> 1) ^ (0xEDB88320u & (0u - (c & 1)));
    }
    return ~c;
}

void put(std::string& s, uint64_t v, int n) { s.append(reinterpret_cast<const char*>(&v), n); }

const uint64_t kExtremes[] = {0, 1, 2, 0x7F, 0x80, 0xFF, 0x7FFF, 0xFFFF, 0x7FFFFFFF, 0x80000000,
                              0xFFFFFFFE, 0xFFFFFFFF, 0x100000000ull, 0x7FFFFFFFFFFFFFFFull,
                              0x8000000000000000ull, 0xFFFFFFFFFFFFFFFEull, 0xFFFFFFFFFFFFFFFFull};
constexpr int kNumExtremes = sizeof kExtremes / sizeof kExtremes[0];

// A stored zip of the records (APPNOTE 4.3.7, 4.3.12, 4.3.16).  With rng,
// one record's central entry moves a random subset of its size and offset
// fields into a zip64 extra field (id 1, APPNOTE 4.5.3) whose values are
// either the true ones or extreme ones.
std::string make_zip(const std::vector<Rec>& recs, Rng* rng = nullptr) {
    std::string body, cd;
    const size_t z64 = rng && !recs.empty() ? rng->below(recs.size()) : (size_t)-1;
    for (size_t ri = 0; ri < recs.size(); ++ri) {
        const Rec& r = recs[ri];
        if (ri == z64) {
            const uint32_t crc = crc32_bytes(r.data), off = (uint32_t)body.size();
            put(body, 0x04034b50u, 4);
            put(body, 20, 2); put(body, 0, 2); put(body, 0, 2); put(body, 0, 2); put(body, 0x21, 2);
            put(body, crc, 4); put(body, r.data.size(), 4); put(body, r.data.size(), 4);
            put(body, r.name.size(), 2); put(body, 0, 2);
            body += r.name + r.data;
            const bool big_u = rng->below(2), big_c = big_u || rng->below(2), big_o = rng->below(2);
            auto val = [&](uint64_t truth) {
                return rng->below(2) ? truth : kExtremes[rng->below(kNumExtremes)];
            };
            std::string extra;
            if (big_u) put(extra, val(r.data.size()), 8);
            if (big_c) put(extra, val(r.data.size()), 8);
            if (big_o) put(extra, val(off), 8);
            if (rng->below(4) == 0 && !extra.empty()) extra.resize(rng->below(extra.size()));
            std::string hdr;
            put(hdr, 1, 2);
            put(hdr, rng->below(8) == 0 ? rng->below(65536) : extra.size(), 2);
            extra = hdr + extra;
            put(cd, 0x02014b50u, 4);
            put(cd, 20, 2); put(cd, 20, 2); put(cd, 0, 2); put(cd, 0, 2); put(cd, 0, 2); put(cd, 0x21, 2);
            put(cd, crc, 4);
            put(cd, big_c ? 0xFFFFFFFFu : r.data.size(), 4);
            put(cd, big_u ? 0xFFFFFFFFu : r.data.size(), 4);
            put(cd, r.name.size(), 2); put(cd, extra.size(), 2); put(cd, 0, 2); put(cd, 0, 2);
            put(cd, 0, 2); put(cd, 0, 4);
            put(cd, big_o ? 0xFFFFFFFFu : off, 4);
            cd += r.name + extra;
            continue;
        }
        const uint32_t crc = crc32_bytes(r.data), off = (uint32_t)body.size();
        put(body, 0x04034b50u, 4);
        put(body, 20, 2); put(body, 0, 2); put(body, 0, 2); put(body, 0, 2); put(body, 0x21, 2);
        put(body, crc, 4); put(body, r.data.size(), 4); put(body, r.data.size(), 4);
        put(body, r.name.size(), 2); put(body, 0, 2);
        body += r.name + r.data;
        put(cd, 0x02014b50u, 4);
        put(cd, 20, 2); put(cd, 20, 2); put(cd, 0, 2); put(cd, 0, 2); put(cd, 0, 2); put(cd, 0x21, 2);
        put(cd, crc, 4); put(cd, r.data.size(), 4); put(cd, r.data.size(), 4);
        put(cd, r.name.size(), 2); put(cd, 0, 2); put(cd, 0, 2); put(cd, 0, 2); put(cd, 0, 2);
        put(cd, 0, 4); put(cd, off, 4);
        cd += r.name;
    }
    std::string z = body + cd;
    put(z, 0x06054b50u, 4); put(z, 0, 2); put(z, 0, 2);
    put(z, recs.size(), 2); put(z, recs.size(), 2);
    put(z, cd.size(), 4); put(z, body.size(), 4); put(z, 0, 2);
    return z;
}

void mutate(std::string& s, Rng& r) {
    const int kinds = 7;
    const int k = (int)r.below(kinds);
    const size_t n = s.size();
    switch (k) {
        case 0:  // flip a bit
            if (n) s[r.below(n)] ^= (char)(1u << r.below(8));
            break;
        case 1:  // set a byte
            if (n) s[r.below(n)] = (char)r.below(256);
            break;
        case 2: {  // an extreme 1/2/4/8-byte value
            const int w = 1 << r.below(4);
            if (n >= (size_t)w) {
                const uint64_t v = kExtremes[r.below(kNumExtremes)];
                std::memcpy(&s[r.below(n - w + 1)], &v, w);
            }
            break;
        }
        case 3:  // truncate
            s.resize(r.below(n + 1));
            break;
        case 4: {  // insert random bytes
            const size_t at = r.below(n + 1), m = 1 + r.below(16);
            std::string ins;
            for (size_t i = 0; i < m; ++i) ins += (char)r.below(256);
            s.insert(at, ins);
            break;
        }
        case 5:  // delete a range
            if (n) {
                const size_t at = r.below(n);
                s.erase(at, 1 + r.below(std::min<size_t>(32, n - at)));
            }
            break;
        default: {  // a field of a zip header (signature PK): an extreme value
            std::vector<size_t> sigs;
            for (size_t i = 0; i + 4 <= n; ++i)
                if (s[i] == 'P' && s[i + 1] == 'K' && (s[i + 2] == 1 || s[i + 2] == 3 ||
                                                       s[i + 2] == 5 || s[i + 2] == 6))
                    sigs.push_back(i);
            if (sigs.empty()) break;
            const size_t at = sigs[r.below(sigs.size())] + 4 + 2 * r.below(22);
            const int w = r.below(2) ? 4 : 2;
            if (at + w <= n) {
                const uint64_t v = kExtremes[r.below(kNumExtremes)];
                std::memcpy(&s[at], &v, w);
            }
        }
    }
}

struct Counts {
    long ok = 0, rejected = 0;
};

// Reads `path` with every reader; each must return 0 or -2.
void read_everything(const std::string& path, Counts& c) {
    int64_t ntok = 0, nslots = 0;
    int has = 0;
    TQStoreFormat fmt;
    int rc = tq_store_read_meta(path.c_str(), &ntok, nullptr, 0, &nslots, &fmt, &has);
    CHECK(rc == 0 || rc == -2);
    if (rc == 0) {
        CHECK(nslots >= 0);
        const int64_t cap = std::min<int64_t>(nslots, 1 << 20);
        std::vector<int32_t> s((size_t)cap + 1);
        rc = tq_store_read_meta(path.c_str(), &ntok, s.data(), cap, &nslots, &fmt, &has);
        CHECK(rc == 0);
    }
    (rc == 0 ? c.ok : c.rejected)++;
    int64_t numel = 0;
    int64_t shape[8];
    int nd = 0;
    rc = tq_store_read_fp16(path.c_str(), &ntok, nullptr, 0, &numel, shape, 8, &nd);
    CHECK(rc == 0 || rc == -2);
    if (rc == 0) {
        CHECK(numel >= 0);
        const int64_t cap = std::min<int64_t>(numel, 1 << 20);
        std::vector<uint16_t> kv((size_t)cap + 1);
        rc = tq_store_read_fp16(path.c_str(), &ntok, kv.data(), cap, &numel, shape, 8, &nd);
        CHECK(rc == 0);
    }
    (rc == 0 ? c.ok : c.rejected)++;
    size_t fb = 0;
    rc = tq_store_pool_info(path.c_str(), &fb, &fmt, &has);
    CHECK(rc == 0 || rc == -2);
}

int run_fuzz(uint64_t seed, long iters, const std::string& dir) {
    // Seeds: two .meta files (with and without the format record), an fp16
    // .bin, a paged .bin with its footer, and a manifest.
    const std::string meta_a = dir + "/seed_a.meta", meta_b = dir + "/seed_b.meta";
    const std::string fp16 = dir + "/seed_c.bin", pool = dir + "/seed_d.bin";
    std::vector<int32_t> sl(37);
    for (int i = 0; i < 37; ++i) sl[i] = 37 - i;
    TQStoreFormat f{1, 1, 2, 128, 16, 4288, 3, 37};
    CHECK(tq_store_write_meta(meta_a.c_str(), 37, sl.data(), 37, &f) == 0);
    CHECK(tq_store_write_meta(meta_b.c_str(), 0, sl.data(), 0, nullptr) == 0);
    std::vector<uint16_t> kv(64, 0x3C00);
    const int64_t shape[3] = {2, 2, 16};
    CHECK(tq_store_write_fp16(fp16.c_str(), 2, kv.data(), 64, shape, 3) == 0);
    std::vector<uint8_t> pages(3 * 4288, 7);
    CHECK(tq_store_write_pool(pool.c_str(), pages.data(), pages.size(), &f) == 0);
    const std::string store = dir + "/store";
    ::mkdir(store.c_str(), 0755);
    CHECK(tq_store_manifest_update(store.c_str(), "doc", 3, "turbo_prod", 37) == 0);
    CHECK(tq_store_manifest_update(store.c_str(), "doc \xce\xb1", 4, "turbo_mse", 5) == 0);
    const std::string manifest = store + "/manifest.json";

    const std::vector<std::string> seeds = {read_all(meta_a), read_all(meta_b), read_all(fp16),
                                            read_all(pool)};
    const std::string mseed = read_all(manifest);
    for (const auto& s : seeds) CHECK(!s.empty());
    Counts c;
    read_everything(meta_a, c);
    CHECK(c.ok >= 1);  // the valid seed reads
    Rng r{seed};
    const std::string path = dir + "/case.meta";
    for (long it = 0; it < iters; ++it) {
        const int which = (int)r.below(7);
        std::string s;
        if (which < 4) {  // a mutated archive
            s = seeds[which];
            for (int m = 1 + (int)r.below(4); m > 0; --m) mutate(s, r);
        } else if (which == 4) {  // a valid archive around a mutated pickle
            auto recs = local_records(seeds[r.below(3)]);
            for (auto& rc : recs)
                if (rc.name.size() >= 8 && rc.name.compare(rc.name.size() - 8, 8, "data.pkl") == 0)
                    for (int m = 1 + (int)r.below(4); m > 0; --m) mutate(rc.data, r);
            s = make_zip(recs);
        } else if (which == 6) {  // zip64 fields in one central entry
            s = make_zip(local_records(seeds[r.below(3)]), &r);
        } else {  // a mutated manifest
            s = mseed;
            for (int m = 1 + (int)r.below(4); m > 0; --m) mutate(s, r);
            write_all(manifest, s);
            const int rc1 = tq_store_manifest_verify(store.c_str(), "doc", 3, "turbo_prod");
            CHECK(rc1 == 0 || rc1 == -2);
            const int rc2 = tq_store_manifest_update(store.c_str(), "doc2", 1, "turbo_prod", 9);
            CHECK(rc2 == 0 || rc2 == -2);
            continue;
        }
        write_all(path, s);
        read_everything(path, c);
    }
    std::printf("fuzz ok: seed %llu, %ld cases, %ld reads accepted, %ld rejected\n",
                (unsigned long long)seed, iters, c.ok, c.rejected);
    return 0;
}

int run_parse(int n, char** files) {
    for (int k = 0; k < n; ++k) {
        int64_t ntok = 0, nslots = 0, numel = 0;
        int has = 0, nd = 0;
        int64_t shape[8];
        const int a = tq_store_read_meta(files[k], &ntok, nullptr, 0, &nslots, nullptr, &has);
        const std::string ea = tq_last_error();
        const int b = tq_store_read_fp16(files[k], &ntok, nullptr, 0, &numel, shape, 8, &nd);
        std::printf("%s meta=%d (%s) fp16=%d (%s)\n", files[k], a, a ? ea.c_str() : "",
                    b, b ? tq_last_error() : "");
        CHECK((a == 0 || a == -2) && (b == 0 || b == -2));
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "abi") == 0) return run_abi();
    if (argc == 5 && std::strcmp(argv[1], "fuzz") == 0)
        return run_fuzz(std::strtoull(argv[2], nullptr, 10), std::strtol(argv[3], nullptr, 10),
                        argv[4]);
    if (argc >= 3 && std::strcmp(argv[1], "parse") == 0) return run_parse(argc - 2, argv + 2);
    std::fprintf(stderr, "usage: host_fuzz abi | fuzz SEED ITERS DIR | parse FILE...\n");
    return 2;
}
