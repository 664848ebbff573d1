// allocator.cpp -- process-global bump allocator on hipMalloc slabs.
//
// Behaviour of nemotron::BumpAllocator (nemotron_infer/csrc/include/tensor/allocator.cuh:58-175):
// 64 MiB slabs (larger when one request needs more), 128-byte aligned blocks, rewind() moves
// the cursor back to slab 0 and keeps every slab so that replaying the same (or a smaller)
// sequence of requests after a rewind touches no hipMalloc, reset() frees all slabs.
// Differences: failures are returned as status codes instead of abort()
// (allocator.cuh:158-163), and the allocator object is never destroyed at process exit (a
// static destructor calling hipFree after the HIP runtime has shut down is unsafe).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <mutex>
#include <vector>

#include "nmi_fp8_linear.h"
#include "nmi_launch.hpp"

namespace nmi {
namespace {

class BumpAllocator {
public:
    static constexpr size_t kSlabBytes = 64ull << 20;
    static constexpr size_t kAlign = 128;

    int allocate(size_t bytes, void** out) {
        std::lock_guard<std::mutex> lock(mu_);
        const size_t need = (std::max<size_t>(bytes, 1) + kAlign - 1) & ~(kAlign - 1);
        if (slabs_.empty() || offset_ + need > slabs_[cur_].size) {
            if (!slabs_.empty() && cur_ + 1 < slabs_.size() && need <= slabs_[cur_ + 1].size) {
                ++cur_;                       // replay after rewind(): reuse the next slab
                offset_ = 0;
            } else {
                void* p = nullptr;
                const size_t sz = std::max(kSlabBytes, need);
                hipError_t e = hipMalloc(&p, sz);
                if (e != hipSuccess) {
                    set_last_error("nmi_alloc: hipMalloc of a %zu-byte slab failed: %s",
                                   sz, hipGetErrorString(e));
                    return (int)e;
                }
                slabs_.push_back(Slab{p, sz});   // as allocator.cuh:164-166
                cur_ = slabs_.size() - 1;
                offset_ = 0;
            }
        }
        *out = static_cast<char*>(slabs_[cur_].ptr) + offset_;
        offset_ += need;
        total_ += need;
        return NMI_OK;
    }

    void rewind() {
        std::lock_guard<std::mutex> lock(mu_);
        cur_ = 0;
        offset_ = 0;
        total_ = 0;
    }

    int reset() {
        std::lock_guard<std::mutex> lock(mu_);
        int rc = NMI_OK;
        for (auto& s : slabs_) {
            hipError_t e = hipFree(s.ptr);
            if (e != hipSuccess && rc == NMI_OK) rc = (int)e;
        }
        slabs_.clear();
        cur_ = offset_ = total_ = 0;
        return rc;
    }

    void stats(size_t* total, size_t* nslabs) {
        std::lock_guard<std::mutex> lock(mu_);
        if (total) *total = total_;
        if (nslabs) *nslabs = slabs_.size();
    }

private:
    struct Slab {
        void* ptr;
        size_t size;
    };
    std::mutex mu_;
    std::vector<Slab> slabs_;
    size_t cur_ = 0, offset_ = 0, total_ = 0;
};

BumpAllocator& global_allocator() {
    static BumpAllocator* a = new BumpAllocator();   // intentionally never destroyed
    return *a;
}

}  // namespace
}  // namespace nmi

extern "C" {

int nmi_alloc(size_t bytes, void** out_ptr) {
    if (!out_ptr) {
        nmi::set_last_error("nmi_alloc: NULL out_ptr");
        return NMI_ERR_INVALID_ARG;
    }
    *out_ptr = nullptr;
    return nmi::global_allocator().allocate(bytes, out_ptr);
}

int nmi_alloc_rewind(void) {
    nmi::global_allocator().rewind();
    return NMI_OK;
}

int nmi_alloc_reset(void) { return nmi::global_allocator().reset(); }

int nmi_alloc_stats(size_t* total_allocated, size_t* num_slabs) {
    nmi::global_allocator().stats(total_allocated, num_slabs);
    return NMI_OK;
}

}  // extern "C"
