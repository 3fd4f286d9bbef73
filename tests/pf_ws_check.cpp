// Host-only check of the prefill workspace bookkeeping (qwengine_amd/csrc/pf_workspace.hpp) with a fake allocator:
// a buffer handed out is never freed before release(), growth keeps the old buffer, release frees each buffer once.
// Built and run by tests/test_pf_workspace.py (no GPU needed).  Exit status 0 = every check passed.
#include <stdio.h>
#include <stdlib.h>

#include <set>

#include "pf_workspace.hpp"

static std::set<void*> g_live;
static int g_freed_twice = 0, g_fail_next = 0;
static char g_arena[1 << 16];
static size_t g_next = 0;

static int fake_alloc(void** p, size_t bytes) {
    (void)bytes;
    if (g_fail_next) {
        g_fail_next = 0;
        return 2;
    }
    *p = g_arena + (g_next++);
    g_live.insert(*p);
    return 0;
}
static int fake_free(void* p) {
    if (g_live.erase(p) != 1) g_freed_twice++;
    return 0;
}
static size_t fake_size(int B, int n_pos) { return (size_t)B * 1000 + (size_t)n_pos; }

#define CHECK(c)                                                  \
    do {                                                          \
        if (!(c)) {                                               \
            fprintf(stderr, "check failed line %d: %s\n", __LINE__, #c); \
            return 1;                                             \
        }                                                         \
    } while (0)

int main() {
    qwa::PfWorkspaces<int (*)(void**, size_t), int (*)(void*), size_t (*)(int, int)> t(fake_alloc, fake_free,
                                                                                          fake_size);
    void* s1 = (void*)0x10;
    void* s2 = (void*)0x20;
    CHECK(t.find(0, s1) == nullptr && !t.covers(nullptr, 1, 1));
    CHECK(t.reserve(0, s1, 512, 4096) == 0);
    qwa::PfSlot* r = t.find(0, s1);
    CHECK(r != nullptr && t.covers(r, 512, 4096) && !t.covers(r, 513, 4096) && !t.covers(r, 512, 4097));
    void* first = r->ptr;
    // a narrower reservation keeps the buffer
    CHECK(t.reserve(0, s1, 256, 2048) == 0 && t.find(0, s1)->ptr == first && t.find(0, s1)->max_B == 512);
    // growth: a new buffer, the old one stays alive (a captured graph may hold it)
    CHECK(t.reserve(0, s1, 1024, 8192) == 0);
    r = t.find(0, s1);
    CHECK(r->ptr != first && g_live.count(first) == 1 && g_live.count(r->ptr) == 1);
    CHECK(r->retired.size() == 1 && r->retired[0] == first && r->max_B == 1024 && r->max_pos == 8192);
    // widening one dimension keeps the other's maximum
    CHECK(t.reserve(0, s1, 64, 16384) == 0);
    r = t.find(0, s1);
    CHECK(r->max_B == 1024 && r->max_pos == 16384 && r->retired.size() == 2);
    // a failed allocation leaves the reservation as it was
    void* cur = r->ptr;
    g_fail_next = 1;
    CHECK(t.reserve(0, s1, 1024, 65536) == 2);
    r = t.find(0, s1);
    CHECK(r->ptr == cur && r->max_pos == 16384 && r->retired.size() == 2);
    // streams and devices are separate slots
    CHECK(t.reserve(0, s2, 128, 1024) == 0 && t.reserve(1, s1, 128, 1024) == 0 && t.count() == 3);
    CHECK(t.find(0, s2)->ptr != t.find(0, s1)->ptr && t.find(1, s1)->ptr != t.find(0, s1)->ptr);
    // nothing was freed so far
    CHECK(g_live.size() == 5 && g_freed_twice == 0);
    // release frees exactly the stream's buffers, each once
    CHECK(t.release(0, s1) == 0 && t.find(0, s1) == nullptr && t.count() == 2);
    CHECK(g_live.size() == 2 && g_freed_twice == 0 && g_live.count(first) == 0);
    CHECK(t.release(0, s1) == 0 && g_freed_twice == 0);  // releasing twice is a no-op
    CHECK(t.release(0, s2) == 0 && t.release(1, s1) == 0 && g_live.empty() && g_freed_twice == 0);
    puts("pf_workspace ok");
    return 0;
}
