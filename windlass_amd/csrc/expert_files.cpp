// expert_files.cpp — the packed-file tier of the expert cache (see
// expert_files.h). Reference I/O path: ExpertCache::init / start_workers /
// worker_loop (src/glm_expert_cache.cuh:139-183,380-475).
//
// Ordering, per task:
//   1. the worker waits for the previous copy out of its pinned buffer
//      (that buffer's event) before pread overwrites it;
//   2. pread the whole record (a short read fails the task);
//   3. its stream waits for the task's gate (recorded on the caller's stream
//      when the slot was resolved: no kernel enqueued before it still reads
//      the slot), copies the record host -> slot (a DMA copy: no kernel runs
//      on the worker's stream, so nothing shares the CUs with the caller's
//      persistent kernels), records the slot's event and the buffer's event;
//   4. the task is marked issued, so wl_cache_get can order the caller's
//      stream after the slot's event (an event not yet recorded would order
//      nothing) and convert the record into the native layout on that stream.
#include "expert_files.h"

#ifndef _GNU_SOURCE
#define _GNU_SOURCE  // O_DIRECT
#endif
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "internal.h"

namespace wl {

static constexpr uint32_t kTaskRing = 256;

std::string FileTier::make_worker(Worker& w) {
    hipError_t e;
    if ((e = hipStreamCreateWithFlags(&w.stream, hipStreamNonBlocking)) != hipSuccess)
        return std::string("io stream: ") + hipGetErrorString(e);
    for (int b = 0; b < 2; b++) {
        if ((e = hipHostMalloc((void**)&w.pinned[b], ref_bytes_, hipHostMallocDefault)) != hipSuccess) {
            w.pinned[b] = nullptr;
            return std::string("pinned io buffer: ") + hipGetErrorString(e);
        }
        if ((e = hipEventCreateWithFlags(&w.buf_ev[b], hipEventDisableTiming)) != hipSuccess)
            return std::string("io event: ") + hipGetErrorString(e);
    }
    if (direct_) {
        void* p = nullptr;
        if (posix_memalign(&p, 4096, ref_bytes_) != 0) return "bounce buffer: out of host memory";
        w.bounce = (uint8_t*)p;
    }
    return "";
}

std::string FileTier::open(const std::string& dir, uint32_t first_layer, uint32_t n_layers, uint32_t n_experts,
                           size_t ref_bytes, uint32_t io_threads, int device, bool direct) {
    first_ = first_layer;
    ref_bytes_ = ref_bytes;
    device_ = device;
    direct_ = direct;
    for (uint32_t l = 0; l < n_layers; l++) {
        char path[4096];
        snprintf(path, sizeof(path), "%s/layer_%u.bin", dir.c_str(), first_layer + l);
        const int fd = ::open(path, O_RDONLY | (direct ? O_DIRECT : 0));
        if (fd < 0) return std::string("open ") + path + ": " + std::strerror(errno);
        fds_.push_back(fd);
        struct stat st;
        if (fstat(fd, &st) != 0) return std::string("stat ") + path + ": " + std::strerror(errno);
        if ((uint64_t)st.st_size < (uint64_t)n_experts * ref_bytes) {
            char msg[4200];
            snprintf(msg, sizeof(msg), "%s holds %lld bytes, fewer than %u records of %zu", path,
                     (long long)st.st_size, n_experts, ref_bytes);
            return msg;
        }
    }
    for (uint32_t i = 0; i < kTaskRing; i++) {
        tasks_.emplace_back(new FileTask());
        free_.push_back(tasks_.back().get());
    }
    if (io_threads == 0) {
        inline_mode_ = true;
        return make_worker(inline_);
    }
    workers_.resize(io_threads);
    for (Worker& w : workers_) {
        const std::string err = make_worker(w);
        if (!err.empty()) return err;
    }
    for (uint32_t i = 0; i < io_threads; i++) threads_.emplace_back([this, i] { loop(i); });
    return "";
}

FileTier::~FileTier() {
    {
        std::lock_guard<std::mutex> lk(qm_);
        stop_ = true;
    }
    qcv_.notify_all();
    for (std::thread& t : threads_)
        if (t.joinable()) t.join();
    auto drop = [](Worker& w) {
        if (w.stream) (void)hipStreamSynchronize(w.stream);
        for (int b = 0; b < 2; b++) {
            if (w.pinned[b]) (void)hipHostFree(w.pinned[b]);
            if (w.buf_ev[b]) (void)hipEventDestroy(w.buf_ev[b]);
        }
        if (w.stream) (void)hipStreamDestroy(w.stream);
        free(w.bounce);
    };
    for (Worker& w : workers_) drop(w);
    drop(inline_);
    for (int fd : fds_)
        if (fd >= 0) ::close(fd);
}

FileTask* FileTier::submit(uint32_t layer, uint32_t expert, uint8_t* dst, hipEvent_t gate, hipEvent_t done) {
    FileTask* t = nullptr;
    {
        std::lock_guard<std::mutex> lk(free_mu_);
        if (free_.empty()) return nullptr;  // every task is queued or unreleased
        t = free_.back();
        free_.pop_back();
    }
    t->fd = fds_[layer];
    t->off = (uint64_t)expert * ref_bytes_;
    t->dst = dst;
    t->gate = gate;
    t->done = done;
    t->layer = layer;
    t->expert = expert;
    t->failed.store(false, std::memory_order_relaxed);
    t->issued.store(false, std::memory_order_relaxed);
    t->why[0] = 0;
    if (inline_mode_) {  // the calling thread is the worker
        if (!run(inline_, t)) t->failed.store(true, std::memory_order_relaxed);
        t->issued.store(true, std::memory_order_release);
        return t;
    }
    {
        std::lock_guard<std::mutex> lk(qm_);
        q_.push_back(t);
    }
    qcv_.notify_one();
    return t;
}

bool FileTier::wait_issued(FileTask* t) {
    std::unique_lock<std::mutex> lk(im_);
    icv_.wait(lk, [t] { return t->issued.load(std::memory_order_acquire); });
    return !t->failed.load(std::memory_order_relaxed);
}

void FileTier::release(FileTask* t) {
    std::lock_guard<std::mutex> lk(free_mu_);
    free_.push_back(t);
}

bool FileTier::run(Worker& w, FileTask* t) {
    const uint32_t b = w.turn;
    w.turn ^= 1u;
    if (w.used[b] && hipEventSynchronize(w.buf_ev[b]) != hipSuccess) {
        snprintf(t->why, sizeof(t->why), "wait for the io buffer failed");
        return false;
    }
    uint8_t* buf = w.bounce ? w.bounce : w.pinned[b];
    size_t got = 0;
    while (got < ref_bytes_) {
        const ssize_t r = ::pread(t->fd, buf + got, ref_bytes_ - got, (off_t)(t->off + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) {
            snprintf(t->why, sizeof(t->why), "pread at %llu: %s", (unsigned long long)(t->off + got),
                     r < 0 ? std::strerror(errno) : "end of file");
            return false;
        }
        got += (size_t)r;
    }
    if (w.bounce) std::memcpy(w.pinned[b], w.bounce, ref_bytes_);
    buf = w.pinned[b];
    auto bad = [t](const char* what) {
        snprintf(t->why, sizeof(t->why), "%s failed", what);
        return false;
    };
    if (t->gate && hipStreamWaitEvent(w.stream, t->gate, 0) != hipSuccess) return bad("gate wait");
    if (hipMemcpyAsync(t->dst, buf, ref_bytes_, hipMemcpyHostToDevice, w.stream) != hipSuccess)
        return bad("host-to-device copy");
    if (hipEventRecord(t->done, w.stream) != hipSuccess) return bad("event record");
    if (hipEventRecord(w.buf_ev[b], w.stream) != hipSuccess) return bad("event record");
    w.used[b] = true;
    return true;
}

void FileTier::loop(uint32_t i) {
    (void)hipSetDevice(device_);  // a new thread starts on device 0
    Worker& w = workers_[i];
    for (;;) {
        FileTask* t = nullptr;
        {
            std::unique_lock<std::mutex> lk(qm_);
            qcv_.wait(lk, [this] { return stop_ || !q_.empty(); });
            if (stop_ && q_.empty()) return;
            t = q_.front();
            q_.pop_front();
        }
        const bool ok = run(w, t);
        {
            std::lock_guard<std::mutex> lk(im_);
            if (!ok) t->failed.store(true, std::memory_order_relaxed);
            t->issued.store(true, std::memory_order_release);
        }
        icv_.notify_all();
    }
}

}  // namespace wl
