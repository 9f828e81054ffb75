// Per-device pools of leased scratch buffers (see workspace.hpp).
#include "workspace.hpp"

#include <mutex>
#include <vector>

namespace bmb {

struct ScratchBuffer {
    void *ptr = nullptr;
    size_t cap = 0;
    // Completes after the last lessee's work: recorded on its stream when it
    // returned the buffer (a created stream), or, for a lessee on the null
    // stream, only when a lease on another stream takes the buffer (`on_null`:
    // the last lessee used the null stream and `done` is not recorded yet).
    hipEvent_t done = nullptr;
    bool recorded = false;
    bool on_null = false;
    hipStream_t last = nullptr;  // the last lessee's stream
};

namespace {
constexpr int MAX_DEVICES = 64;

struct Pool {
    std::mutex mu;
    std::vector<ScratchBuffer *> idle;  // buffers not leased right now
};

// Never destroyed: a thread may still return a lease while the process exits.
Pool &pool(int dev, ScratchSlot slot) {
    static Pool *pools = new Pool[MAX_DEVICES * SCRATCH_SLOTS];
    return pools[dev * SCRATCH_SLOTS + slot];
}
}  // namespace

ScratchLease::ScratchLease(ScratchSlot slot, size_t bytes, hipStream_t stream)
    : slot_(slot), stream_(stream) {
    int dev = 0;
    if (slot < 0 || slot >= SCRATCH_SLOTS) return;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        (void)hipGetLastError();
        return;
    }
    if (bytes == 0) bytes = 256;
    Pool &p = pool(dev, slot);
    {
        // The smallest idle buffer that fits and was last used on this
        // stream (no wait on another stream's work); else the smallest that
        // fits; else the largest idle one, to grow; else a new one.
        std::lock_guard<std::mutex> lock(p.mu);
        int same = -1, fit = -1, big = -1;
        for (int i = 0; i < (int)p.idle.size(); ++i) {
            const size_t c = p.idle[i]->cap;
            if (c >= bytes && p.idle[i]->last == stream &&
                (same < 0 || c < p.idle[same]->cap))
                same = i;
            if (c >= bytes && (fit < 0 || c < p.idle[fit]->cap)) fit = i;
            if (big < 0 || c > p.idle[big]->cap) big = i;
        }
        const int pick = same >= 0 ? same : fit >= 0 ? fit : big;
        if (pick >= 0) {
            buf_ = p.idle[pick];
            p.idle.erase(p.idle.begin() + pick);
        } else {
            buf_ = new ScratchBuffer;
        }
    }
    dev_ = dev;
    // The event only orders device work on one device (a later lessee's
    // kernels after an earlier one's), so it needs no system-scope fence: a
    // fenced event costs about 3 us of device time per record, one without it
    // about 1.5.
    if (buf_->done == nullptr &&
        hipEventCreateWithFlags(&buf_->done, hipEventDisableTiming | hipEventDisableSystemFence) !=
            hipSuccess) {
        (void)hipGetLastError();
        buf_->done = nullptr;
        return;  // no way to order reuse: no buffer (the destructor puts it back)
    }
    const bool grow = buf_->cap < bytes;
    if (buf_->on_null && (grow || stream_ != nullptr)) {
        // The last lessee's work is on the null stream, queued before
        // anything queued there from now on: an event recorded there now
        // completes after it.
        if (hipEventRecord(buf_->done, nullptr) != hipSuccess) {
            (void)hipGetLastError();
            return;
        }
        buf_->recorded = true;
        buf_->on_null = false;
    }
    if (grow) {
        if (buf_->ptr != nullptr) {
            // Work queued by an earlier lessee may still read the old buffer.
            if (buf_->recorded && hipEventSynchronize(buf_->done) != hipSuccess) {
                (void)hipGetLastError();
                return;
            }
            (void)hipFree(buf_->ptr);
            buf_->ptr = nullptr;
            buf_->cap = 0;
        }
        void *q = nullptr;
        if (hipMalloc(&q, bytes) != hipSuccess) {
            (void)hipGetLastError();  // clear the allocation failure
            return;
        }
        buf_->ptr = q;
        buf_->cap = bytes;
    } else if (buf_->recorded && hipStreamWaitEvent(stream_, buf_->done, 0) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    // (on_null left set: this lessee is on the null stream too, where its
    // work runs after the last lessee's in queue order.)
    ptr_ = buf_->ptr;
}

ScratchLease::~ScratchLease() {
    if (buf_ == nullptr) return;
    if (ptr_ != nullptr && stream_ == nullptr) {
        // The null stream is never destroyed: the event is recorded there only
        // when a lease on another stream takes the buffer (one record per call
        // saved for the common case of back-to-back calls on the null stream).
        buf_->on_null = true;
        buf_->recorded = false;
        buf_->last = nullptr;
    } else if (ptr_ != nullptr) {
        // After everything this lease's caller queued on its stream (recorded
        // now: the caller may destroy its stream).
        if (hipEventRecord(buf_->done, stream_) == hipSuccess) {
            buf_->recorded = true;
            buf_->on_null = false;
            buf_->last = stream_;
        } else {
            (void)hipGetLastError();
            // Unordered reuse is not allowed: wait for the stream instead.
            if (hipStreamSynchronize(stream_) != hipSuccess) (void)hipGetLastError();
            buf_->recorded = false;
        }
    }
    Pool &p = pool(dev_, slot_);
    std::lock_guard<std::mutex> lock(p.mu);
    p.idle.push_back(buf_);
}

}  // namespace bmb
