// Bookkeeping of the per-(device, stream) prefill workspaces behind the drop-in attn_prefill (host code only; the
// allocator is a template parameter so that the rules can be tested without a GPU).
//
// Rules:
//  * a workspace, once handed to a kernel, is never freed before release(): a HIP graph that captured a prefill
//    keeps its pointer, so growing a reservation allocates a new buffer and keeps the old one alive ("retired")
//    until the stream's release();
//  * lookups and growth happen under the caller's lock, and the caller keeps that lock until its kernels are
//    enqueued, so a concurrent release() (which synchronises the stream before freeing) cannot free a buffer
//    between its lookup and its launch;
//  * covers(B, n_pos) is true when B <= max_B and n_pos <= max_pos and the buffer holds size(B, n_pos) bytes.
#pragma once

#include <stddef.h>

#include <algorithm>
#include <vector>

namespace qwa {

struct PfSlot {
    int dev;
    void* stream;
    void* ptr;       // current workspace
    size_t bytes;
    int max_B;
    int max_pos;
    std::vector<void*> retired;  // earlier, smaller workspaces of this stream, alive until release
};

// Alloc: int alloc(void** p, size_t bytes) -> 0 on success; Free: int free(void* p) -> 0 on success;
// Size: size_t size(int B, int n_pos).
template <class Alloc, class Free, class Size>
class PfWorkspaces {
public:
    PfWorkspaces(Alloc a, Free f, Size s) : alloc_(a), free_(f), size_(s) {}

    PfSlot* find(int dev, void* stream) {
        for (auto& r : slots_)
            if (r.dev == dev && r.stream == stream) return &r;
        return nullptr;
    }

    bool covers(const PfSlot* r, int B, int n_pos) const {
        return r != nullptr && B <= r->max_B && n_pos <= r->max_pos && size_(B, n_pos) <= r->bytes;
    }

    // Widens (dev, stream)'s reservation to cover B <= max_B, n_pos <= max_pos as well as what it covered before.
    // Returns 0, or the allocator's error (the reservation is then unchanged).
    int reserve(int dev, void* stream, int max_B, int max_pos) {
        PfSlot* r = find(dev, stream);
        if (r != nullptr) {
            max_B = std::max(r->max_B, max_B);
            max_pos = std::max(r->max_pos, max_pos);
        }
        const size_t need = size_(max_B, max_pos);
        if (r != nullptr && r->bytes >= need) {
            r->max_B = max_B;
            r->max_pos = max_pos;
            return 0;
        }
        void* p = nullptr;
        if (int e = alloc_(&p, need)) return e;
        if (r != nullptr) {
            r->retired.push_back(r->ptr);  // a captured graph may still use it
            r->ptr = p;
            r->bytes = need;
            r->max_B = max_B;
            r->max_pos = max_pos;
        } else {
            slots_.push_back(PfSlot{dev, stream, p, need, max_B, max_pos, {}});
        }
        return 0;
    }

    // Removes (dev, stream)'s reservation and frees its buffers; the caller has synchronised the stream first.
    // Returns 0 or the first free error (every buffer is still freed).
    int release(int dev, void* stream) {
        for (size_t i = 0; i < slots_.size(); i++) {
            if (slots_[i].dev == dev && slots_[i].stream == stream) {
                int err = free_(slots_[i].ptr);
                for (void* p : slots_[i].retired) {
                    const int e = free_(p);
                    if (err == 0) err = e;
                }
                slots_.erase(slots_.begin() + (long)i);
                return err;
            }
        }
        return 0;
    }

    size_t count() const { return slots_.size(); }

private:
    Alloc alloc_;
    Free free_;
    Size size_;
    std::vector<PfSlot> slots_;
};

}  // namespace qwa
