// A minimal litemind::ThreadPool (interface of include/Threading.hpp:16-41) for
// programs built against the drop-in headers alone.
#include "Threading.hpp"

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

namespace litemind {

struct ThreadPool::State {};

ThreadPool::ThreadPool(std::size_t worker_count)
    : worker_count_(worker_count == 0U ? hardware_threads() : worker_count) {}

ThreadPool::~ThreadPool() = default;

void ThreadPool::parallel_for(std::size_t count, const std::function<void(std::size_t)>& body) {
    const std::size_t workers = std::min(worker_count_, count);
    if (workers <= 1U) {
        for (std::size_t i = 0; i < count; ++i) {
            body(i);
        }
        return;
    }
    std::atomic<std::size_t> next{0};
    std::vector<std::thread> threads;
    threads.reserve(workers - 1U);
    auto run = [&] {
        for (std::size_t i = next.fetch_add(1); i < count; i = next.fetch_add(1)) {
            body(i);
        }
    };
    for (std::size_t w = 1; w < workers; ++w) {
        threads.emplace_back(run);
    }
    run();
    for (std::thread& t : threads) {
        t.join();
    }
}

std::size_t ThreadPool::hardware_threads() noexcept {
    const unsigned n = std::thread::hardware_concurrency();
    return n == 0U ? 1U : static_cast<std::size_t>(n);
}

}  // namespace litemind
