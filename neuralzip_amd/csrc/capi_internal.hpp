// capi_internal.hpp -- helpers shared by the extern "C" translation units.
#pragma once
#include <algorithm>
#include <atomic>
#include <exception>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "codebook.hpp"
#include "codec.hpp"

struct nz_codebook {
    nz::Codebook book;       // token lengths, GPU canonical codes, LUT image
    nz::Huff0Tables huff;    // storage code of Huff0 headers (unused for NZM1)
};

namespace nz_capi {

int set_error(int code, const char* message);

template <typename F>
int guarded(F&& body) {
    try {
        body();
        return 0;
    } catch (const nz::Error& e) {
        return set_error(e.code, e.what());
    } catch (const std::bad_alloc&) {
        return set_error(nz::kOutOfMemory, "Out of host memory.");
    } catch (const std::exception& e) {
        return set_error(nz::kInvalidArgument, e.what());
    } catch (...) {
        return set_error(nz::kInvalidArgument, "Unknown native failure.");
    }
}

// run_parallel_jobs (neuralzip/native/common.h:134-185): at most 16
// workers (hardware concurrency by default), one below 512 KiB of input;
// every job runs, and the first failing job's error is rethrown.
template <typename Job>
void parallel_for(size_t count, size_t total_bytes, int threads, Job&& job) {
    if (count == 0) return;
    const unsigned hw = std::thread::hardware_concurrency();
    int workers = threads > 0 ? threads : static_cast<int>(hw ? hw : 1);
    workers = std::max(1, std::min<int>({workers, 16, static_cast<int>(std::min<size_t>(count, 1 << 20))}));
    if (total_bytes < (512u << 10)) workers = 1;
    std::vector<std::string> errors(count);
    std::vector<int> codes(count, 0);
    std::atomic<size_t> next{0};
    auto worker = [&]() {
        for (size_t i; (i = next.fetch_add(1)) < count;) {
            try {
                job(i);
            } catch (const nz::Error& e) {
                errors[i] = e.what();
                codes[i] = e.code;
            } catch (const std::exception& e) {
                errors[i] = e.what();
                codes[i] = nz::kInvalidArgument;
            }
        }
    };
    if (workers == 1) {
        worker();
    } else {
        std::vector<std::thread> pool;
        for (int w = 0; w < workers; ++w) pool.emplace_back(worker);
        for (auto& t : pool) t.join();
    }
    for (size_t i = 0; i < count; ++i)
        if (codes[i]) throw nz::Error(codes[i], errors[i]);
}

}  // namespace nz_capi
