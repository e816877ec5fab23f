// Minimal LuisaCompute-shaped host runtime over HIP, enough for the LCPP device hot path:
// Device, Stream, CommandList (recorded closures run in order on commit), Buffer<T> / BufferView<T>,
// DoubleBuffer<T> and the temp-storage helpers.  Shapes follow the reference's usage
// (README.md:160-190; e.g. tests/device_radix_sort_interface_test.cpp:95-145):
//   auto buf = device.create_buffer<uint>(n);
//   CommandList cmd; radix_sort.SortKeys(cmd, temp.view(), in.view(), out.view(), n);
//   stream << in.copy_from(host.data()) << cmd.commit() << out.copy_to(result.data()) << synchronize();
// All device work goes through HIP on one stream; nothing runs before commit.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <span>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "lcpp_hip.h"

namespace luisa {

using uint = uint32_t;
using ulong = uint64_t;
using slong = int64_t;

template <typename T>
using vector = std::vector<T>;
using string = std::string;
using std::span;  // luisa::span{v} deduces like the reference's luisa::span

// Errors raised by the facade (the reference aborts through LUISA_ASSERT on the same conditions).
class Error : public std::runtime_error {
  public:
    using std::runtime_error::runtime_error;
};

namespace detail {
inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}
inline void abi_check(int status, const char* what) {
    if (status != LCPP_HIP_OK) throw Error(std::string(what) + ": " + lcpp_hip_last_error());
}
}  // namespace detail

#define LCPP_ASSERT(cond, msg)                                  \
    do {                                                        \
        if (!(cond)) throw ::luisa::Error(std::string(msg));   \
    } while (0)

namespace compute {

using luisa::uint;
using luisa::ulong;

// A device command: runs on the stream it is submitted to.
using Command = std::function<void(hipStream_t)>;

template <typename T>
class BufferView {
  public:
    BufferView() = default;
    BufferView(T* data, size_t size) : m_data(data), m_size(size) {}
    [[nodiscard]] T* data() const noexcept { return m_data; }
    [[nodiscard]] size_t size() const noexcept { return m_size; }
    [[nodiscard]] size_t size_bytes() const noexcept { return m_size * sizeof(T); }
    [[nodiscard]] BufferView subview(size_t offset, size_t count) const {
        LCPP_ASSERT(offset + count <= m_size, "BufferView::subview out of range");
        return BufferView(m_data + offset, count);
    }
    // Reinterprets the bytes of this view as elements of U (size rounded down).
    template <typename U>
    [[nodiscard]] BufferView<U> as() const {
        return BufferView<U>(reinterpret_cast<U*>(m_data), m_size * sizeof(T) / sizeof(U));
    }
    [[nodiscard]] Command copy_from(const void* host) const {
        T* d = m_data;
        size_t b = size_bytes();
        return [d, b, host](hipStream_t s) {
            if (b) detail::hip_check(hipMemcpyAsync(d, host, b, hipMemcpyHostToDevice, s), "copy_from");
        };
    }
    template <typename U, size_t E>
    [[nodiscard]] Command copy_from(std::span<U, E> host) const {
        LCPP_ASSERT(host.size_bytes() >= size_bytes(), "BufferView::copy_from: host span is smaller than the view");
        return copy_from(static_cast<const void*>(host.data()));
    }
    [[nodiscard]] Command copy_from(BufferView<T> src) const {
        T* d = m_data;
        const T* sp = src.data();
        size_t b = size_bytes();
        return [d, sp, b](hipStream_t s) {
            if (b) detail::hip_check(hipMemcpyAsync(d, sp, b, hipMemcpyDeviceToDevice, s), "copy_from(view)");
        };
    }
    [[nodiscard]] Command copy_to(void* host) const {
        const T* d = m_data;
        size_t b = size_bytes();
        return [d, b, host](hipStream_t s) {
            if (b) detail::hip_check(hipMemcpyAsync(host, d, b, hipMemcpyDeviceToHost, s), "copy_to");
        };
    }
    template <typename U, size_t E>
    [[nodiscard]] Command copy_to(std::span<U, E> host) const {
        LCPP_ASSERT(host.size_bytes() >= size_bytes(), "BufferView::copy_to: host span is smaller than the view");
        return copy_to(static_cast<void*>(host.data()));
    }

  private:
    T* m_data = nullptr;
    size_t m_size = 0;
};

template <typename T>
class Buffer {
  public:
    Buffer() = default;
    explicit Buffer(size_t n) : m_size(n) {
        if (n) {
            void* p = nullptr;
            detail::hip_check(hipMalloc(&p, n * sizeof(T)), "hipMalloc");
            m_data.reset(static_cast<T*>(p));
        }
    }
    [[nodiscard]] BufferView<T> view() const { return BufferView<T>(m_data.get(), m_size); }
    [[nodiscard]] BufferView<T> view(size_t offset, size_t count) const { return view().subview(offset, count); }
    [[nodiscard]] size_t size() const noexcept { return m_size; }
    [[nodiscard]] T* data() const noexcept { return m_data.get(); }
    template <typename Src>
    [[nodiscard]] Command copy_from(Src&& src) const { return view().copy_from(std::forward<Src>(src)); }
    template <typename Dst>
    [[nodiscard]] Command copy_to(Dst&& dst) const { return view().copy_to(std::forward<Dst>(dst)); }
    operator BufferView<T>() const { return view(); }

  private:
    struct Free {
        void operator()(T* p) const noexcept { (void)hipFree(p); }
    };
    std::unique_ptr<T, Free> m_data;
    size_t m_size = 0;
};

// Marker: `stream << synchronize()` waits for all submitted work.
struct SynchronizeToken {};
inline SynchronizeToken synchronize() { return {}; }

// Recorded commands; `commit()` hands them to a stream in recording order.
class CommandList {
  public:
    CommandList& operator<<(Command c) {
        m_commands.push_back(std::move(c));
        return *this;
    }
    CommandList& add(Command c) { return *this << std::move(c); }
    [[nodiscard]] bool empty() const noexcept { return m_commands.empty(); }
    [[nodiscard]] size_t size() const noexcept { return m_commands.size(); }
    // Moves the recorded commands out; the list is empty afterwards.
    [[nodiscard]] Command commit() {
        auto cmds = std::make_shared<std::vector<Command>>(std::move(m_commands));
        m_commands.clear();
        return [cmds](hipStream_t s) {
            for (auto& c : *cmds) c(s);
        };
    }

  private:
    std::vector<Command> m_commands;
};

class Stream {
  public:
    Stream() = default;
    explicit Stream(int device) : m_device(device) {
        detail::hip_check(hipSetDevice(device), "hipSetDevice");
        hipStream_t s = nullptr;
        detail::hip_check(hipStreamCreate(&s), "hipStreamCreate");
        m_stream = std::shared_ptr<std::remove_pointer_t<hipStream_t>>(s, [](hipStream_t p) { (void)hipStreamDestroy(p); });
    }
    [[nodiscard]] hipStream_t handle() const noexcept { return m_stream.get(); }
    Stream& operator<<(const Command& c) {
        c(handle());
        return *this;
    }
    Stream& operator<<(SynchronizeToken) {
        detail::hip_check(hipStreamSynchronize(handle()), "hipStreamSynchronize");
        return *this;
    }
    void synchronize() { *this << compute::synchronize(); }

  private:
    int m_device = 0;
    std::shared_ptr<std::remove_pointer_t<hipStream_t>> m_stream;
};

class Device {
  public:
    Device() = default;
    explicit Device(int ordinal) : m_ordinal(ordinal) {}
    [[nodiscard]] int ordinal() const noexcept { return m_ordinal; }
    [[nodiscard]] std::string backend_name() const { return "hip"; }
    template <typename T>
    [[nodiscard]] Buffer<T> create_buffer(size_t n) const {
        detail::hip_check(hipSetDevice(m_ordinal), "hipSetDevice");
        return Buffer<T>(n);
    }
    [[nodiscard]] Stream create_stream() const { return Stream(m_ordinal); }

  private:
    int m_ordinal = 0;
};

// Entry point mirroring LuisaCompute's Context (only the HIP device exists here).
class Context {
  public:
    Context() = default;
    explicit Context(const std::string&) {}
    [[nodiscard]] Device create_device(const std::string& = "hip", int ordinal = 0) const { return Device(ordinal); }
};

}  // namespace compute

namespace parallel_primitive {

using namespace luisa::compute;

// Not used on this backend; present so that create(device, stream, nullptr) keeps compiling.
class InteropContext;

// common/util_type.h:16-60: a pair of buffers and the index of the current one.
template <typename T>
struct DoubleBuffer {
    BufferView<T> d_buffer[2];
    int selector = 0;
    DoubleBuffer() = default;
    DoubleBuffer(BufferView<T> current, BufferView<T> alternate) : d_buffer{current, alternate}, selector(0) {}
    [[nodiscard]] BufferView<T> current() const { return d_buffer[selector & 1]; }
    [[nodiscard]] BufferView<T> alternate() const { return d_buffer[(selector & 1) ^ 1]; }
};

// common/utils.h:247-250.
inline size_t bytes_to_uint_count(size_t byte_size) { return (byte_size + sizeof(uint) - 1) / sizeof(uint); }

// common/thread_operators.h:49-74: the sum, max and min operators accepted by the scan entry points.
// On the device, float min / max ignore a NaN operand (fmin / fmax).
struct SumOp {
    template <typename T>
    T operator()(const T& a, const T& b) const { return a + b; }
};
struct MaxOp {
    template <typename T>
    T operator()(const T& a, const T& b) const { return b > a ? b : a; }
};
struct MinOp {
    template <typename T>
    T operator()(const T& a, const T& b) const { return b < a ? b : a; }
};

// Transforms of DeviceReduce::TransformReduce.  The reference takes any device callable
// (common/thread_operators.h:76-84 IdentityOp); the C-ABI's fixed vocabulary covers its tests: the
// identity, scale * x + shift, x * x and |x| (integers wrap, floats round after every operation).
struct IdentityOp {
    template <typename T>
    T operator()(const T& x) const { return x; }
};
template <typename T>
struct AffineOp {
    T scale, shift;
    T operator()(const T& x) const { return scale * x + shift; }
};
struct SquareOp {
    template <typename T>
    T operator()(const T& x) const { return x * x; }
};
struct AbsOp {
    template <typename T>
    T operator()(const T& x) const { return x < T(0) ? T(0) - x : x; }
};

template <typename T>
concept NumericT = std::is_integral_v<T> || std::is_floating_point_v<T>;  // common/type_trait.h:14

// runtime/core.h:69-112: every module is created against a device before dispatch.
class LuisaModule {
  protected:
    Device m_device;
    bool m_created = false;
    void create_module(Device& device) {
        m_device = device;
        m_created = true;
    }
};

namespace detail {
inline void* stream_ptr(hipStream_t s) { return static_cast<void*>(s); }
}  // namespace detail

}  // namespace parallel_primitive
}  // namespace luisa
