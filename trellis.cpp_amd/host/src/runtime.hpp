// Internal interface of the HIP graph runtime behind the ggml-compatible headers: device memory
// RAII, ggml <-> library dtype mapping, the elementwise kernels' launchers (ggml_ops.hip) and
// the context hooks the sparse adapter uses to keep per-graph state alive.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <exception>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "ggml-backend.h"
#include "ggml.h"
#include "trellis_sparse.h"

namespace tgr {

constexpr size_t kAlign = 256;
inline size_t align_up(size_t x, size_t a = kAlign) { return (x + a - 1) / a * a; }

[[noreturn]] void fail(const std::string& msg);   // throws std::runtime_error
void hip_check(hipError_t e, const char* what);    // throws on error

// Owning device allocation on the current device. The stream-ordered form takes a block from a
// cache kept per (device, stream) and gives it back there when it goes out of scope, without a
// synchronisation: the block is only handed out again to a later allocation on the same stream,
// whose work runs after everything queued before the release. Blocks come from hipMalloc and stay
// cached until the process ends; an allocation that finds the device full first synchronises the
// device and frees the cached blocks. (HIP's stream-ordered pool, hipMallocAsync / hipFreeAsync,
// is not used: under the decoders' allocation pattern its calls blocked the host for 0.1-5 s at
// times.)
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes);
    DeviceBuffer(size_t bytes, hipStream_t s);
    ~DeviceBuffer();
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept
        : p_(o.p_), n_(o.n_), cap_(o.cap_), s_(o.s_), dev_(o.dev_), mode_(o.mode_) {
        o.p_ = nullptr;
        o.n_ = o.cap_ = 0;
    }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            reset();
            p_ = o.p_;
            n_ = o.n_;
            cap_ = o.cap_;
            s_ = o.s_;
            dev_ = o.dev_;
            mode_ = o.mode_;
            o.p_ = nullptr;
            o.n_ = o.cap_ = 0;
        }
        return *this;
    }
    void reset();
    void* get() const { return p_; }
    template <class T> T* as() const { return static_cast<T*>(p_); }
    size_t size() const { return n_; }

private:
    enum Mode { kPlain, kCached };
    void* p_ = nullptr;
    size_t n_ = 0;     // bytes asked for
    size_t cap_ = 0;   // bytes of the cached block
    hipStream_t s_ = nullptr;
    int dev_ = 0;
    Mode mode_ = kPlain;
};

// Device -> host copy of `bytes` at src, stream-ordered on s, through two pinned staging
// buffers (kept until the process ends): while the host takes one chunk (sink(ptr, n), in
// order), the next one is in flight.
void download_chunks(const void* src, size_t bytes, hipStream_t s,
                     const std::function<void(const void*, size_t)>& sink);

// Asks the kernel to back [p, p + bytes) with huge pages (a hint; first touches of a large fresh
// buffer otherwise fault one 4 KiB page at a time).
void advise_huge_pages(void* p, size_t bytes);

// Device -> host copy of `bytes` at src into host memory at dst, stream-ordered on s: each staged
// chunk is copied out by several host threads. dst should be touched memory (see HostVector).
void download_into(void* dst, const void* src, size_t bytes, hipStream_t s);

// download_into for a buffer whose contents are produced chunk by chunk: produce(off, len)
// enqueues on s the work that writes bytes [off, off + len) of src (in order; chunks of whole
// units of `unit` bytes but the last), and each chunk is copied, on a stream of its own, while the
// next one is produced.
void download_produced(void* dst, const void* src, size_t bytes, size_t unit, hipStream_t s,
                       const std::function<void(size_t, size_t)>& produce);

// A host vector of `count` value-initialised elements, made on a thread of its own: the first
// touches of a large fresh buffer (page faults, the kernel zeroing the pages) then overlap with
// device work queued before the result is needed. take() waits for the thread and hands the
// vector over (rethrowing what the thread threw).
template <class T>
class HostVector {
public:
    HostVector() = default;
    explicit HostVector(size_t count) { start(count); }
    HostVector(const HostVector&) = delete;
    HostVector& operator=(const HostVector&) = delete;
    ~HostVector() {
        if (th_.joinable()) th_.join();
    }
    void start(size_t count) {
        if (th_.joinable()) th_.join();
        th_ = std::thread([this, count] {
            try {
                v_.clear();
                v_.reserve(count);
                advise_huge_pages(v_.data(), count * sizeof(T));
                v_.resize(count);
            } catch (...) {
                err_ = std::current_exception();
            }
        });
    }
    std::vector<T> take() {
        if (th_.joinable()) th_.join();
        if (err_) std::rethrow_exception(err_);
        return std::move(v_);
    }

private:
    std::vector<T> v_;
    std::thread th_;
    std::exception_ptr err_;
};

// count elements of device memory at src into a new host vector (no zero-fill first).
template <class T>
std::vector<T> download(const void* src, size_t count, hipStream_t s) {
    std::vector<T> v;
    v.reserve(count);
    advise_huge_pages(v.data(), count * sizeof(T));
    download_chunks(src, count * sizeof(T), s, [&](const void* p, size_t n) {
        const T* t = static_cast<const T*>(p);
        v.insert(v.end(), t, t + n / sizeof(T));
    });
    return v;
}

// HIP device and stream of a backend made by ggml_backend_hip_init.
int backend_device(ggml_backend_t backend);
hipStream_t backend_stream(ggml_backend_t backend);

// Library dtype of a floating ggml type; -1 for the others.
int tsp_dtype_of(enum ggml_type t);
bool is_contiguous(const ggml_tensor* t);

// The context owns `obj` until ggml_free.
void context_keep(ggml_context* ctx, std::shared_ptr<void> obj);
// Per-context memo (e.g. the conv plan node of a neighbour table).
ggml_tensor* context_memo_get(ggml_context* ctx, const ggml_tensor* key, int kind);
void context_memo_put(ggml_context* ctx, const ggml_tensor* key, int kind, ggml_tensor* value);

// Elementwise kernels (ggml_ops.hip); all return hipSuccess or the launch error.
// out = a (op) b with b broadcast over a (ggml_can_repeat); a/b f32 or f16, out f32.
hipError_t launch_binary(int op_mul, const ggml_tensor* a, const ggml_tensor* b, float* out,
                         hipStream_t s);
hipError_t launch_silu(const float* x, float* y, int64_t n, hipStream_t s);
// y[i] = (y_dtype) silu(x[i]) for a 16-bit y
hipError_t launch_silu_to(const float* x, void* y, int y_dtype, int64_t n, hipStream_t s);
// y[i] += x[i] (x f32 / f16 / bf16)
hipError_t launch_add_inplace(float* y, const void* x, int x_dtype, int64_t n, hipStream_t s);
// y[i] = (dtype) x[i]: f32 -> f16 / bf16 (round to nearest even), and f16 / bf16 -> f32.
hipError_t launch_convert(const void* x, int x_dtype, void* y, int y_dtype, int64_t n,
                          hipStream_t s);
// The decoders' head: out [n][co] f32 = LN(eps, no affine)(x [n][ci] f32) . W^T + bias, W [co][ci]
// of w_dtype, bias f32 [co]; co <= 8, ci in {16, 32, 64, 128, 256, 512, 1024}, x 16-byte aligned
// (hipErrorInvalidValue otherwise: the caller takes the two-pass route).
hipError_t launch_norm_linear(const float* x, int64_t n, int ci, float eps, const void* w, int w_dtype,
                              const float* bias, int co, float* out, hipStream_t s);
// out[r][k] = a[idx[r]][k] for a [rows][k] (f32/f16/i32 -> f32, i32 -> i32).
hipError_t launch_get_rows(const ggml_tensor* a, const int32_t* idx, int64_t n_idx, void* out,
                           hipStream_t s);

}  // namespace tgr
