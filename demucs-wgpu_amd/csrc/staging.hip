// staging.hip — HostPool, host_copy_async, prefault_async and PinnedRing
// (declared in staging.h): the host side of the runner's transfers.
#include "staging.h"

#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "common.h"

namespace dmx {

namespace {
constexpr size_t PAGE = 4096;
constexpr size_t HUGE_PAGE = 2u << 20;
// Below this a copy is not split: a part costs a wake-up (~10 us).
constexpr size_t MIN_PART = 512u << 10;

int pool_threads() {
    if (const char *v = std::getenv("DMX_HOST_THREADS")) {
        int n = std::atoi(v);
        if (n >= 0) return std::min(n, 64);
    }
    unsigned hw = std::thread::hardware_concurrency();
    return (int)std::min<unsigned>(8, hw ? hw : 1);
}

// [lo, hi) of part `i` of `parts` over n bytes, page aligned.
void part_range(size_t n, int i, int parts, size_t &lo, size_t &hi) {
    size_t per = (n / (size_t)parts + PAGE - 1) / PAGE * PAGE;
    lo = std::min(n, per * (size_t)i);
    hi = std::min(n, lo + per);
}
}  // namespace

HostPool &HostPool::instance() {
    // Never destroyed: the workers sleep on the condition variable until the
    // process ends, so no static-destruction order can stop them mid-job.
    static HostPool *pool = new HostPool();
    return *pool;
}

HostPool::HostPool() {
    const int n = pool_threads();
    for (int i = 0; i < n; ++i) workers_.emplace_back([this] { worker(); });
    for (auto &t : workers_) t.detach();
}

uint64_t HostPool::submit(Body body, int parts) {
    parts = std::max(parts, 1);
    std::unique_lock<std::mutex> lock(mu_);
    Job *j = new Job{next_id_++, std::move(body), parts, 0, parts};
    queue_.push_back(j);
    open_.insert(j->id);
    lock.unlock();
    if (parts == 1)
        work_cv_.notify_one();
    else
        work_cv_.notify_all();
    return j->id;
}

// Claims the next part of the oldest job (if its id <= upto) and runs it
// with the lock released. Returns false when there was nothing to claim.
bool HostPool::run_one(std::unique_lock<std::mutex> &lock, uint64_t upto) {
    if (queue_.empty() || queue_.front()->id > upto) return false;
    Job *j = queue_.front();
    const int part = j->next++;
    if (j->next == j->parts) queue_.pop_front();
    lock.unlock();
    j->body(part, j->parts);
    lock.lock();
    if (--j->left == 0) {
        open_.erase(j->id);
        delete j;
        done_cv_.notify_all();
    }
    return true;
}

void HostPool::worker() {
    std::unique_lock<std::mutex> lock(mu_);
    for (;;) {
        work_cv_.wait(lock, [this] { return !queue_.empty(); });
        run_one(lock, UINT64_MAX);
    }
}

void HostPool::wait(uint64_t ticket) {
    std::unique_lock<std::mutex> lock(mu_);
    while (open_.count(ticket))
        if (!run_one(lock, ticket)) done_cv_.wait(lock);
}

uint64_t host_copy_async(void *dst, const void *src, size_t n) {
    HostPool &pool = HostPool::instance();
    const int parts = (int)std::max<size_t>(1, std::min<size_t>(pool.threads() + 1, n / MIN_PART));
    char *d = static_cast<char *>(dst);
    const char *s = static_cast<const char *>(src);
    return pool.submit(
        [=](int i, int k) {
            size_t lo, hi;
            part_range(n, i, k, lo, hi);
            if (hi > lo) std::memcpy(d + lo, s + lo, hi - lo);
        },
        parts);
}

uint64_t prefault_async(void *p, size_t n) {
    HostPool &pool = HostPool::instance();
    char *base = static_cast<char *>(p);
    advise_huge_pages(p, n);
    const int parts = (int)std::max<size_t>(1, std::min<size_t>(pool.threads(), n / (4 * HUGE_PAGE)));
    return pool.submit(
        [=](int i, int k) {
            size_t lo, hi;
            part_range(n, i, k, lo, hi);
            // Writing a byte's own value maps the page writable and keeps
            // the caller's data.
            for (size_t off = lo; off < hi; off += PAGE) {
                volatile char *q = base + off;
                *q = *q;
            }
        },
        parts);
}

uint64_t host_copy_ranges_async(std::vector<Copy> copies) {
    HostPool &pool = HostPool::instance();
    size_t total = 0;
    for (const Copy &c : copies) total += c.bytes;
    const int parts = (int)std::max<size_t>(1, std::min<size_t>(pool.threads() + 1, total / MIN_PART));
    // Part i copies bytes [lo, hi) of the ranges laid end to end.
    return pool.submit(
        [copies = std::move(copies), total](int i, int k) {
            size_t lo, hi;
            part_range(total, i, k, lo, hi);
            size_t at = 0;
            for (const Copy &c : copies) {
                const size_t a = std::max(lo, at), b = std::min(hi, at + c.bytes);
                if (b > a)
                    std::memcpy(static_cast<char *>(c.dst) + (a - at), static_cast<const char *>(c.src) + (a - at),
                                b - a);
                at += c.bytes;
                if (at >= hi) break;
            }
        },
        parts);
}

EventCopier::EventCopier(int device, std::vector<uint64_t> before)
    : device_(device), before_(std::move(before)), thread_([this] { run(); }) {}

EventCopier::~EventCopier() {
    try {
        finish();
    } catch (...) {
    }
}

void EventCopier::push(hipEvent_t ev, std::vector<Copy> copies) {
    {
        std::lock_guard<std::mutex> lock(mu_);
        tasks_.push_back({ev, std::move(copies)});
    }
    cv_.notify_one();
}

void EventCopier::finish() {
    {
        std::lock_guard<std::mutex> lock(mu_);
        closed_ = true;
    }
    cv_.notify_one();
    if (thread_.joinable()) thread_.join();
    if (!error_.empty()) {
        std::string msg;
        msg.swap(error_);
        throw_error(6, msg);
    }
}

void EventCopier::run() {
    const bool device_ok = hipSetDevice(device_) == hipSuccess;
    for (;;) {
        Task t;
        {
            std::unique_lock<std::mutex> lock(mu_);
            cv_.wait(lock, [this] { return closed_ || !tasks_.empty(); });
            if (tasks_.empty()) return;
            t = std::move(tasks_.front());
            tasks_.pop_front();
        }
        // After a failure the rest of the queue is dropped: its host memory
        // may not hold what the device wrote.
        if (!error_.empty()) continue;
        if (!device_ok) {
            error_ = "readback thread: hipSetDevice(" + std::to_string(device_) + ") failed";
            continue;
        }
        const hipError_t e = hipEventSynchronize(t.ev);
        if (e != hipSuccess) {
            error_ = std::string("readback thread: hipEventSynchronize failed: ") + hipGetErrorString(e);
            continue;
        }
        for (uint64_t b : before_) HostPool::instance().wait(b);
        before_.clear();
        HostPool::instance().wait(host_copy_ranges_async(std::move(t.copies)));
    }
}

PinnedRing::~PinnedRing() {
    for (hipEvent_t e : ev_)
        if (e) {
            (void)hipEventSynchronize(e);
            (void)hipEventDestroy(e);
        }
    if (mem_) (void)hipHostFree(mem_);
}

void PinnedRing::ensure() {
    if (mem_) return;
    for (hipEvent_t &e : ev_) DMX_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    DMX_HIP(hipHostMalloc((void **)&mem_, (size_t)SLOTS * SLOT_BYTES, hipHostMallocDefault));
}

std::vector<PinnedRing::Piece> PinnedRing::pieces(const std::vector<Span> &spans) {
    std::vector<Piece> out;
    for (const Span &s : spans)
        for (size_t off = 0; off < s.bytes; off += SLOT_BYTES)
            out.push_back({static_cast<char *>(s.dev) + off, static_cast<char *>(s.host) + off,
                           std::min(SLOT_BYTES, s.bytes - off)});
    return out;
}

void PinnedRing::upload(const std::vector<Span> &spans, hipStream_t stream) {
    ensure();
    const std::vector<Piece> ps = pieces(spans);
    for (size_t i = 0; i < ps.size(); ++i) {
        const int k = (int)(i % SLOTS);
        char *slot = mem_ + (size_t)k * SLOT_BYTES;
        // The slot's previous DMA (upload or download) has to be done.
        DMX_HIP(hipEventSynchronize(ev_[k]));
        host_copy(slot, ps[i].host, ps[i].bytes);
        DMX_HIP(hipMemcpyAsync(ps[i].dev, slot, ps[i].bytes, hipMemcpyHostToDevice, stream));
        DMX_HIP(hipEventRecord(ev_[k], stream));
    }
}

void PinnedRing::download(const std::vector<Span> &spans, hipStream_t stream) {
    ensure();
    const std::vector<Piece> ps = pieces(spans);
    if (ps.empty()) return;
    // Piece i goes through slot i % SLOTS, and its host copy starts `lag`
    // pieces later, so that many DMAs stay in flight meanwhile. A copy is
    // waited for one iteration after it starts; with lag = SLOTS - 2 the
    // copy out of slot (i - SLOTS) % SLOTS has ended before piece i's DMA
    // refills it.
    const size_t lag = SLOTS - 2;
    uint64_t pending = 0;
    try {
        for (size_t i = 0; i < ps.size() + lag; ++i) {
            if (i < ps.size()) {
                const int k = (int)(i % SLOTS);
                DMX_HIP(hipMemcpyAsync(mem_ + (size_t)k * SLOT_BYTES, ps[i].dev, ps[i].bytes, hipMemcpyDeviceToHost,
                                       stream));
                DMX_HIP(hipEventRecord(ev_[k], stream));
            }
            if (i >= lag) {
                const size_t j = i - lag;
                const int k = (int)(j % SLOTS);
                DMX_HIP(hipEventSynchronize(ev_[k]));
                if (pending) HostPool::instance().wait(pending);
                pending = 0;
                pending = host_copy_async(ps[j].host, mem_ + (size_t)k * SLOT_BYTES, ps[j].bytes);
            }
        }
    } catch (...) {
        // No host copy may outlive the call that owns its destination.
        if (pending) HostPool::instance().wait(pending);
        (void)hipStreamSynchronize(stream);
        throw;
    }
    if (pending) HostPool::instance().wait(pending);
}

PinnedBuffer::~PinnedBuffer() {
    if (mem_) (void)hipHostFree(mem_);
}

char *PinnedBuffer::reserve(size_t bytes) {
    if (bytes <= bytes_) return mem_;
    if (mem_) DMX_HIP(hipHostFree(mem_));
    mem_ = nullptr;
    bytes_ = 0;
    DMX_HIP(hipHostMalloc((void **)&mem_, bytes, hipHostMallocDefault));
    bytes_ = bytes;
    return mem_;
}

void advise_huge_pages(void *p, size_t n) {
    char *base = static_cast<char *>(p);
    uintptr_t a = ((uintptr_t)base + HUGE_PAGE - 1) & ~(uintptr_t)(HUGE_PAGE - 1);
    uintptr_t b = ((uintptr_t)base + n) & ~(uintptr_t)(HUGE_PAGE - 1);
    if (b > a) (void)madvise(reinterpret_cast<void *>(a), b - a, MADV_HUGEPAGE);
}

}  // namespace dmx
