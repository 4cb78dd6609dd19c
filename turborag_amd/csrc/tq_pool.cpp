// tq_pool.cpp — page allocator and block table (host bookkeeping).
//
// TQAllocator follows src/tq_allocator.cpp:5-31: one device pool of
// num_pages * page_size bytes, a LIFO free list initialised [N-1 ... 0] so
// pages come out 0, 1, 2, ..., alloc -> -1 when empty, free pushes back.
// TQBlockTable follows src/tq_block_table.cpp:4-43: per-sequence page list,
// slots phys*block_size + tib, pages allocated on demand, "out of blocks"
// when the allocator runs dry.  Unlike the reference, a failed append leaves
// the sequence unchanged (pages taken for it are returned).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>
#include <new>
#include <unordered_map>
#include <vector>

#include "tq_internal.h"

struct TQAllocator {
    size_t page_size = 0;
    int num_pages = 0;
    uint8_t* pool = nullptr;
    bool owned = false;
    std::vector<int32_t> free_list;
    mutable std::mutex mu;
};

struct TQBlockTable {
    struct Seq {
        std::vector<int32_t> blocks;
        int num_tokens = 0;
    };
    TQAllocator* alloc = nullptr;
    int block_size = 16;
    std::unordered_map<int32_t, Seq> seqs;
    mutable std::mutex mu;
};

namespace {
int fail(const char* msg) {
    tq::set_last_error(msg);
    return -2;
}
}  // namespace

extern "C" int tq_allocator_create(size_t page_size_bytes, int num_pages, uint8_t* device_pool,
                                   TQAllocator** out) {
    if (!out) return -1;
    if (num_pages < 0 || page_size_bytes == 0) return fail("tq_allocator_create: bad size");
    TQAllocator* a = new (std::nothrow) TQAllocator();
    if (!a) return fail("tq_allocator_create: out of host memory");
    a->page_size = page_size_bytes;
    a->num_pages = num_pages;
    if (device_pool) {
        a->pool = device_pool;
    } else if (num_pages > 0) {
        void* p = nullptr;
        if (hipMalloc(&p, page_size_bytes * (size_t)num_pages) != hipSuccess) {
            (void)hipGetLastError();
            delete a;
            return fail("hipMalloc page_pool failed");
        }
        a->pool = static_cast<uint8_t*>(p);
        a->owned = true;
    }
    a->free_list.reserve((size_t)num_pages);
    for (int i = num_pages - 1; i >= 0; --i) a->free_list.push_back(i);
    *out = a;
    return 0;
}

extern "C" int tq_allocator_destroy(TQAllocator* a) {
    if (!a) return -1;
    if (a->owned && a->pool) (void)hipFree(a->pool);
    delete a;
    return 0;
}

extern "C" int tq_allocator_alloc_block(TQAllocator* a, int32_t* out_block) {
    if (!a || !out_block) return -1;
    std::lock_guard<std::mutex> lock(a->mu);
    if (a->free_list.empty()) {
        *out_block = -1;
        return 0;
    }
    *out_block = a->free_list.back();
    a->free_list.pop_back();
    return 0;
}

extern "C" int tq_allocator_free_block(TQAllocator* a, int32_t block) {
    if (!a) return -1;
    if (block < 0 || block >= a->num_pages) return fail("tq_allocator_free_block: bad page id");
    std::lock_guard<std::mutex> lock(a->mu);
    a->free_list.push_back(block);
    return 0;
}

extern "C" int tq_allocator_num_free(const TQAllocator* a, int* out) {
    if (!a || !out) return -1;
    std::lock_guard<std::mutex> lock(a->mu);
    *out = (int)a->free_list.size();
    return 0;
}

extern "C" uint8_t* tq_allocator_device_pool(const TQAllocator* a) { return a ? a->pool : nullptr; }

extern "C" int tq_block_table_create(TQAllocator* a, int block_size, TQBlockTable** out) {
    if (!a || !out) return -1;
    if (block_size <= 0) return fail("tq_block_table_create: block_size must be > 0");
    TQBlockTable* t = new (std::nothrow) TQBlockTable();
    if (!t) return fail("tq_block_table_create: out of host memory");
    t->alloc = a;
    t->block_size = block_size;
    *out = t;
    return 0;
}

extern "C" int tq_block_table_destroy(TQBlockTable* t) {
    if (!t) return -1;
    delete t;
    return 0;
}

extern "C" int tq_block_table_build_slot_map(TQBlockTable* t, int32_t seq_id, int append_tokens,
                                             int32_t* out_slots) {
    if (!t || (!out_slots && append_tokens > 0)) return -1;
    if (append_tokens < 0) return fail("tq_block_table_build_slot_map: append_tokens < 0");
    std::lock_guard<std::mutex> lock(t->mu);
    TQBlockTable::Seq& s = t->seqs[seq_id];
    const int bs = t->block_size;
    const int old_blocks = (s.num_tokens + bs - 1) / bs;
    const int new_blocks = (s.num_tokens + append_tokens + bs - 1) / bs;
    std::vector<int32_t> fresh;
    for (int i = old_blocks; i < new_blocks; ++i) {
        int32_t b = -1;
        tq_allocator_alloc_block(t->alloc, &b);
        if (b < 0) {
            for (auto it = fresh.rbegin(); it != fresh.rend(); ++it)
                tq_allocator_free_block(t->alloc, *it);
            return fail("out of blocks");
        }
        fresh.push_back(b);
    }
    s.blocks.insert(s.blocks.end(), fresh.begin(), fresh.end());
    for (int i = 0; i < append_tokens; ++i) {
        const int tok = s.num_tokens + i;
        out_slots[i] = s.blocks[(size_t)(tok / bs)] * bs + tok % bs;
    }
    s.num_tokens += append_tokens;
    return 0;
}

extern "C" int tq_block_table_num_tokens(const TQBlockTable* t, int32_t seq_id, int* out) {
    if (!t || !out) return -1;
    std::lock_guard<std::mutex> lock(t->mu);
    auto it = t->seqs.find(seq_id);
    if (it == t->seqs.end()) return fail("tq_block_table: unknown sequence");
    *out = it->second.num_tokens;
    return 0;
}

extern "C" int tq_block_table_blocks(const TQBlockTable* t, int32_t seq_id, int32_t* out_blocks,
                                     int capacity, int* out_num_blocks) {
    if (!t || !out_num_blocks || (!out_blocks && capacity > 0)) return -1;
    std::lock_guard<std::mutex> lock(t->mu);
    auto it = t->seqs.find(seq_id);
    if (it == t->seqs.end()) return fail("tq_block_table: unknown sequence");
    const auto& b = it->second.blocks;
    for (int i = 0; i < capacity && i < (int)b.size(); ++i) out_blocks[i] = b[(size_t)i];
    *out_num_blocks = (int)b.size();
    return 0;
}

extern "C" int tq_block_table_free_sequence(TQBlockTable* t, int32_t seq_id) {
    if (!t) return -1;
    std::lock_guard<std::mutex> lock(t->mu);
    auto it = t->seqs.find(seq_id);
    if (it == t->seqs.end()) return fail("tq_block_table: unknown sequence");
    for (int32_t b : it->second.blocks) tq_allocator_free_block(t->alloc, b);
    t->seqs.erase(it);
    return 0;
}
