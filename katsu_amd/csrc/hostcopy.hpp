// hostcopy.hpp -- copies between the caller's pageable host buffers and the
// device for the host-pointer entry points (the drop-in seams, whose Rust
// callers hand over `&[f32]` slices, tensor.rs:172-174).
//
// A pageable buffer cannot be read by the GPU's DMA engines directly, so a
// copy is staged through pinned host memory.  Here the staging is a ring of
// kSlots pinned chunks of chunk_ bytes owned by the library: the CPU copy of
// one chunk into (or out of) the ring overlaps the DMA of the others, and the
// CPU copy is itself split over a few threads, since one core copies well
// below the PCIe rate.  Each chunk's DMA is ordered on the caller's stream
// and followed by an event; a slot is refilled only after its event has
// completed.  Small copies, and every copy when pinned memory cannot be had,
// go through hipMemcpyAsync on the pageable buffer.  Four slots of 8 MiB
// (KATSU_COPY_CHUNK_MB) and four copying threads (KATSU_COPY_THREADS) are
// the measured defaults: a config-3 step through the host seams takes about
// 4.0 ms against 6.4-7.0 ms through HIP's own pageable copies; one thread
// copies too slowly (6-7 ms), and more than four, or chunks of 4 or 16 MiB,
// gave no further gain.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace katsu {

// A memcpy split over the calling thread and up to kMaxThreads - 1 helper
// threads that live until the process ends (the pool is never destroyed, so
// no thread outlives what it touches).  The job and its part counter are
// read and updated under the pool's mutex, so a helper that wakes late can
// only take a part of the job still open.  One copy at a time: callers hold
// the library mutex.
class CopyPool {
  public:
    static CopyPool &get() {
        static CopyPool *p = new CopyPool();
        return *p;
    }

    void copy(void *dst, const void *src, size_t n) {
        const int parts = (int)std::min<size_t>(nthreads_, std::max<size_t>(1, n >> 20));
        if (parts <= 1) {
            std::memcpy(dst, src, n);
            return;
        }
        std::unique_lock<std::mutex> lk(mu_);
        dst_ = (char *)dst;
        src_ = (const char *)src;
        n_ = n;
        parts_ = parts;
        next_ = 0;
        finished_ = 0;
        ++gen_;
        work_cv_.notify_all();
        run_parts(lk);
        done_cv_.wait(lk, [&] { return finished_ == parts_; });
    }

  private:
    CopyPool() {
        const char *env = std::getenv("KATSU_COPY_THREADS");
        const int t = env ? std::atoi(env) : kDefaultThreads;
        nthreads_ = std::max(1, std::min(t, kMaxThreads));
        for (int i = 1; i < nthreads_; ++i) std::thread([this] { loop(); }).detach();
    }

    // Takes parts of the open job until none is left (lk held on entry and
    // exit).  Parts are whole 4 KiB pages.
    void run_parts(std::unique_lock<std::mutex> &lk) {
        while (next_ < parts_) {
            const int k = next_++;
            const size_t per = ((n_ / parts_) + 4095) & ~(size_t)4095;
            const size_t b = std::min(n_, (size_t)k * per), e = std::min(n_, b + per);
            char *d = dst_;
            const char *s = src_;
            lk.unlock();
            if (e > b) std::memcpy(d + b, s + b, e - b);
            lk.lock();
            if (++finished_ == parts_) done_cv_.notify_all();
        }
    }

    void loop() {
        std::unique_lock<std::mutex> lk(mu_);
        uint64_t seen = gen_;
        for (;;) {
            work_cv_.wait(lk, [&] { return gen_ != seen; });
            seen = gen_;
            run_parts(lk);
        }
    }

    static constexpr int kDefaultThreads = 4, kMaxThreads = 16;
    int nthreads_ = 1;
    std::mutex mu_;
    std::condition_variable work_cv_, done_cv_;
    uint64_t gen_ = 0;
    int next_ = 0, finished_ = 0, parts_ = 0;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t n_ = 0;
};

class HostCopy {
  public:
    static constexpr int kSlots = 4;
    static constexpr size_t kDirectBelow = 1u << 20;  // smaller copies skip the ring

    // Host to device, ordered on `st`.  The caller's buffer must stay as it
    // is until the entry point's final synchronisation (the seams' inputs are
    // immutable for the call).
    hipError_t h2d(void *dst, const void *src, size_t bytes, hipStream_t st) {
        if (bytes < kDirectBelow || !ring())
            return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
        for (size_t off = 0, i = 0; off < bytes; off += chunk_, ++i) {
            const size_t len = std::min(chunk_, bytes - off);
            const int slot = (int)(i % kSlots);
            hipError_t e = wait_slot(slot);
            if (e != hipSuccess) return e;
            CopyPool::get().copy(pinned_[slot], (const char *)src + off, len);
            e = hipMemcpyAsync((char *)dst + off, pinned_[slot], len, hipMemcpyHostToDevice, st);
            if (e == hipSuccess) e = record(slot, st);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }

    // Device to host after the work already ordered on `st`; returns when the
    // caller's buffer holds the data.
    hipError_t d2h(void *dst, const void *src, size_t bytes, hipStream_t st) {
        if (bytes < kDirectBelow || !ring()) {
            const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st);
            return e != hipSuccess ? e : hipStreamSynchronize(st);
        }
        const size_t nchunk = (bytes + chunk_ - 1) / chunk_;
        auto issue = [&](size_t i) {
            const int slot = (int)(i % kSlots);
            hipError_t e = wait_slot(slot);
            if (e != hipSuccess) return e;
            const size_t off = i * chunk_, len = std::min(chunk_, bytes - off);
            e = hipMemcpyAsync(pinned_[slot], (const char *)src + off, len,
                               hipMemcpyDeviceToHost, st);
            return e == hipSuccess ? record(slot, st) : e;
        };
        for (size_t i = 0; i < std::min<size_t>(nchunk, kSlots); ++i) {
            const hipError_t e = issue(i);
            if (e != hipSuccess) return e;
        }
        for (size_t i = 0; i < nchunk; ++i) {
            const int slot = (int)(i % kSlots);
            hipError_t e = wait_slot(slot);
            if (e != hipSuccess) return e;
            const size_t off = i * chunk_, len = std::min(chunk_, bytes - off);
            CopyPool::get().copy((char *)dst + off, pinned_[slot], len);
            if (i + kSlots < nchunk && (e = issue(i + kSlots)) != hipSuccess) return e;
        }
        return hipSuccess;
    }

    // Waits for the ring's last DMAs and frees it (library shutdown).
    void release() {
        for (int i = 0; i < kSlots; ++i) {
            if (busy_[i]) (void)hipEventSynchronize(ev_[i]);
            busy_[i] = false;
            if (ev_[i]) (void)hipEventDestroy(ev_[i]);
            if (pinned_[i]) (void)hipHostFree(pinned_[i]);
            ev_[i] = nullptr;
            pinned_[i] = nullptr;
        }
        tried_ = false;
    }

  private:
    // The pinned ring, allocated on first use; false when it cannot be had.
    bool ring() {
        if (!tried_) {
            tried_ = true;
            if (const char *env = std::getenv("KATSU_COPY_CHUNK_MB"))
                chunk_ = (size_t)std::max(1, std::min(std::atoi(env), 64)) << 20;
            bool ok = true;
            for (int i = 0; i < kSlots && ok; ++i) {
                ok = hipHostMalloc(&pinned_[i], chunk_, hipHostMallocDefault) == hipSuccess &&
                     hipEventCreateWithFlags(&ev_[i], hipEventDisableTiming) == hipSuccess;
            }
            if (!ok) {
                (void)hipGetLastError();
                release();
                tried_ = true;
            }
        }
        return pinned_[kSlots - 1] != nullptr && ev_[kSlots - 1] != nullptr;
    }
    // Polls the slot's event: a chunk's DMA takes about 75 us, and a blocking
    // wait adds a wake-up latency of the same order to each of them.
    hipError_t wait_slot(int slot) {
        if (!busy_[slot]) return hipSuccess;
        busy_[slot] = false;
        hipError_t e;
        while ((e = hipEventQuery(ev_[slot])) == hipErrorNotReady) {
        }
        return e;
    }
    hipError_t record(int slot, hipStream_t st) {
        const hipError_t e = hipEventRecord(ev_[slot], st);
        busy_[slot] = e == hipSuccess;
        return e;
    }

    void *pinned_[kSlots] = {};
    hipEvent_t ev_[kSlots] = {};
    bool busy_[kSlots] = {};
    bool tried_ = false;
    size_t chunk_ = 8u << 20;  // KATSU_COPY_CHUNK_MB overrides (1-64)
};

}  // namespace katsu
