// expert_files.h — the packed-file tier of the expert cache: misses read from
// `dir`/layer_N.bin (the reference's packed expert files: 256 records of one
// reference-layout expert block each, record e at e x block bytes;
// tools/repack_experts_glm.py:5-14,46-55) by a pool of pread workers, each
// with two pinned host buffers and a non-blocking stream, and copied as they
// are (reference layout) into the slot; the cache converts a slot into the
// native layout on the caller's stream when it first hands it out (reference
// I/O path: src/glm_expert_cache.cuh:29-62,339-475). Host-only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <condition_variable>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace wl {

// One block read: record `expert` of file `layer` into device slot `dst`
// (the record's bytes as they are in the file).
struct FileTask {
    int fd = -1;
    uint64_t off = 0;
    uint8_t* dst = nullptr;
    hipEvent_t gate = nullptr;  // the copy waits for it (no kernel still reads the slot)
    hipEvent_t done = nullptr;  // recorded after the block landed in dst (the slot's event)
    uint32_t layer = 0, expert = 0;
    std::atomic<bool> issued{false};  // the worker has recorded `done` (or failed)
    std::atomic<bool> failed{false};
    char why[96] = {0};               // the failure, set before `issued`
};

class FileTier {
public:
    // Opens dir/layer_{first_layer + l}.bin for l < n_layers and checks that
    // each holds n_experts records of ref_bytes; starts io_threads workers
    // (0: every read runs on the calling thread). direct: O_DIRECT reads
    // (ref_bytes a multiple of 4096) into a page-aligned bounce buffer per
    // worker, copied into the pinned buffer. Returns an empty string or an
    // error message.
    std::string open(const std::string& dir, uint32_t first_layer, uint32_t n_layers, uint32_t n_experts,
                     size_t ref_bytes, uint32_t io_threads, int device, bool direct = false);
    ~FileTier();

    // Queues the read of (layer, expert) into dst; the copy waits for `gate`
    // and records `done` once the block is in place. The task is owned by the
    // tier and stays valid until the next submit that reuses it (a ring of
    // tasks, reused once issued and released).
    FileTask* submit(uint32_t layer, uint32_t expert, uint8_t* dst, hipEvent_t gate, hipEvent_t done);
    // Blocks until the task is issued; false if its read failed.
    bool wait_issued(FileTask* t);
    // Releases a task for reuse (after wait_issued).
    void release(FileTask* t);
    uint32_t first_layer() const { return first_; }
    size_t ref_bytes() const { return ref_bytes_; }

private:
    struct Worker {
        hipStream_t stream = nullptr;
        uint8_t* pinned[2] = {nullptr, nullptr};
        uint8_t* bounce = nullptr;  // direct mode: page-aligned ordinary memory the O_DIRECT reads land in
                                    // (direct I/O into the runtime's pinned mappings fails with EFAULT)
        hipEvent_t buf_ev[2] = {nullptr, nullptr};
        bool used[2] = {false, false};
        uint32_t turn = 0;
    };
    std::string make_worker(Worker& w);
    void loop(uint32_t i);
    bool run(Worker& w, FileTask* t);  // read, copy, record; false on a short read

    std::vector<int> fds_;
    uint32_t first_ = 0;
    size_t ref_bytes_ = 0;
    int device_ = 0;
    std::vector<std::unique_ptr<FileTask>> tasks_;
    std::vector<FileTask*> free_;
    std::mutex free_mu_;
    std::vector<Worker> workers_;
    Worker inline_;  // io_threads == 0
    bool inline_mode_ = false;
    bool direct_ = false;
    std::vector<std::thread> threads_;
    std::deque<FileTask*> q_;
    std::mutex qm_;
    std::condition_variable qcv_;
    std::mutex im_;
    std::condition_variable icv_;
    bool stop_ = false;
};

}  // namespace wl
