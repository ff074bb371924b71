#pragma once
// litemind::ThreadPool's interface (include/Threading.hpp:16-41).  The GPU
// drop-in does no CPU fan-out: gemm:: accepts the pool for signature
// compatibility and runs on the device.  This small pool exists so programs built
// against these headers alone (the demo) can construct one; inside LiteMind its
// own Threading.cpp is used.

#include <cstddef>
#include <functional>

namespace litemind {

class ThreadPool final {
public:
    explicit ThreadPool(std::size_t worker_count = 0U);
    ~ThreadPool();

    ThreadPool(const ThreadPool&) = delete;
    ThreadPool& operator=(const ThreadPool&) = delete;

    void parallel_for(std::size_t count, const std::function<void(std::size_t)>& body);

    [[nodiscard]] std::size_t worker_count() const noexcept { return worker_count_; }
    [[nodiscard]] static std::size_t hardware_threads() noexcept;

private:
    struct State;

    std::size_t worker_count_{1U};
    State* state_{nullptr};
};

}  // namespace litemind
