// staging.h — the host side of the runner's transfers: a small pool of host
// threads for copies between pinned staging memory and the caller's arrays,
// and a ring of pinned slots that pipelines host copies with DMA.
//
// Measured on the MI355X box: pinned DMA runs at ~57 GB/s each way; one host
// thread copies ~30 GB/s into memory that is already mapped but under
// 2 GB/s into a freshly allocated array, whose first write to each page
// faults; eight threads on huge pages copy into fresh memory at ~50 GB/s.
// So a caller's output array is pre-faulted (huge-page advised, one write of
// its own value per page) by the pool while the GPU computes, and every
// large host copy is split over the pool's threads.
#pragma once

#include <hip/hip_runtime.h>

#include <condition_variable>
#include <cstdint>
#include <deque>
#include <functional>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <vector>

namespace dmx {

// Process-wide worker threads running parallel-for jobs. A job is a body
// called once per part (part, parts); jobs start in submission order, and a
// thread that waits for a job runs unclaimed parts of it (and of older jobs)
// itself. Threads: DMX_HOST_THREADS, else min(8, hardware threads).
class HostPool {
  public:
    using Body = std::function<void(int part, int parts)>;
    static HostPool &instance();
    int threads() const { return (int)workers_.size(); }
    uint64_t submit(Body body, int parts);
    void wait(uint64_t ticket);
    void run(Body body, int parts) { wait(submit(std::move(body), parts)); }

  private:
    struct Job {
        uint64_t id;
        Body body;
        int parts, next, left;
    };
    HostPool();
    void worker();
    bool run_one(std::unique_lock<std::mutex> &lock, uint64_t upto);
    std::mutex mu_;
    std::condition_variable work_cv_, done_cv_;
    std::deque<Job *> queue_;  // jobs with unclaimed parts, oldest first
    std::set<uint64_t> open_;  // jobs not finished
    uint64_t next_id_ = 1;
    std::vector<std::thread> workers_;
};

// dst[0, n) = src[0, n) on the pool (asynchronous; wait on the ticket).
uint64_t host_copy_async(void *dst, const void *src, size_t n);
inline void host_copy(void *dst, const void *src, size_t n) { HostPool::instance().wait(host_copy_async(dst, src, n)); }

// Asks for huge pages over the 2 MB-aligned interior of [p, p + n) of the
// caller's memory (advice only: a kernel that refuses it keeps 4 KB pages).
void advise_huge_pages(void *p, size_t n);

// Maps every page of [p, p + n) for writing without changing its contents,
// on huge pages where the kernel allows them (asynchronous).
uint64_t prefault_async(void *p, size_t n);

// One host-to-host copy.
struct Copy {
    void *dst;
    const void *src;
    size_t bytes;
};

// Every range of `copies` on the pool as one job, split evenly by bytes
// (asynchronous; wait on the ticket).
uint64_t host_copy_ranges_async(std::vector<Copy> copies);

// Host copies that wait for device events, run from a thread of its own: the
// caller queues (event, copies) pairs in order while it goes on enqueueing
// GPU work, and each pair's copies start on the pool as soon as its event has
// completed. finish() (also run by the destructor) returns when every queued
// copy is done and reports the first failure as a dmx::Error. The pool jobs
// in `before` (e.g. the prefault of the same destination pages) end before
// the first copy starts.
class EventCopier {
  public:
    EventCopier(int device, std::vector<uint64_t> before);
    EventCopier(const EventCopier &) = delete;
    EventCopier &operator=(const EventCopier &) = delete;
    ~EventCopier();
    void push(hipEvent_t ev, std::vector<Copy> copies);
    void finish();

  private:
    struct Task {
        hipEvent_t ev;
        std::vector<Copy> copies;
    };
    void run();
    int device_;
    std::vector<uint64_t> before_;
    std::mutex mu_;
    std::condition_variable cv_;
    std::deque<Task> tasks_;
    bool closed_ = false;
    std::string error_;
    std::thread thread_;
};

// One contiguous range moved between host and device memory.
struct Span {
    void *dev;
    void *host;
    size_t bytes;
};

// A ring of pinned slots through which host ranges move to and from the
// device on a caller's stream; host copies of one slot overlap the DMA of
// the others. Owned by one runner and used by one thread at a time.
//
// The copies go on the runner's own stream, not a stream of their own: with
// GPU_MAX_HW_QUEUES = 4 (the HIP default) a fifth stream shares a hardware
// queue with a busy one and its copies wait behind that queue's kernels.
class PinnedRing {
  public:
    static constexpr int SLOTS = 6;
    static constexpr size_t SLOT_BYTES = 4u << 20;
    PinnedRing() = default;
    PinnedRing(const PinnedRing &) = delete;
    PinnedRing &operator=(const PinnedRing &) = delete;
    ~PinnedRing();
    // host -> device on `stream`. Returns once every host byte has been read.
    void upload(const std::vector<Span> &spans, hipStream_t stream);
    // device -> host on `stream`, after the work already queued on it.
    // Returns when every byte is in host memory.
    void download(const std::vector<Span> &spans, hipStream_t stream);

  private:
    struct Piece {
        char *dev, *host;
        size_t bytes;
    };
    void ensure();
    static std::vector<Piece> pieces(const std::vector<Span> &spans);
    char *mem_ = nullptr;
    hipEvent_t ev_[SLOTS] = {};
};

// Pinned host memory that grows to the largest size asked for (and is kept).
class PinnedBuffer {
  public:
    PinnedBuffer() = default;
    PinnedBuffer(const PinnedBuffer &) = delete;
    PinnedBuffer &operator=(const PinnedBuffer &) = delete;
    ~PinnedBuffer();
    // At least `bytes`; the device must not be using the old memory.
    char *reserve(size_t bytes);

  private:
    char *mem_ = nullptr;
    size_t bytes_ = 0;
};

}  // namespace dmx
