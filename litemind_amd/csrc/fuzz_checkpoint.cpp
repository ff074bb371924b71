// fuzz_checkpoint.cpp -- mutation fuzzer of the SafeTensors reader (lm_checkpoint.cpp)
// for a CPU build with AddressSanitizer and UndefinedBehaviorSanitizer.
//
//   fuzz_checkpoint <work_dir> <iterations> <seed> <seed_file>...
//
// Each iteration takes one seed file, applies a few random mutations (bit and
// byte flips, truncation, insertion of JSON fragments, a rewritten header
// length), writes it as <work_dir>/model.safetensors and runs the reader's
// entry points over it: lm_checkpoint_open, then lm_checkpoint_count and, for
// a few tensor names, lm_checkpoint_find / _require / _read_f32, and
// lm_checkpoint_close.  Every call must return (an error status is fine); the
// sanitizers turn an out-of-bounds access, a use after free or undefined
// behaviour into a failing exit.  The GPU entry points the reader's layer
// loader calls are not used here and are stubbed.
#include "litemind_moe.h"
#include "lm_error.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

namespace {
thread_local std::string g_message;
}

int lm::set_error(int code, const std::string& message) {
    g_message = message;
    return code;
}

extern "C" {
// Stubs of the GPU half of the ABI (lm_load_layer / lm_load_head call them).
int lm_context_config(lm_context*, lm_moe_config*) { return LM_EINVAL; }
int lm_upload_router(lm_context*, int32_t, const float*) { return LM_EINVAL; }
int lm_upload_expert(lm_context*, int32_t, int32_t, const uint16_t*, const uint16_t*, const uint16_t*) { return LM_EINVAL; }
int lm_upload_shared(lm_context*, int32_t, const uint16_t*, const uint16_t*, const uint16_t*) { return LM_EINVAL; }
int lm_upload_dense(lm_context*, int32_t, const uint16_t*, const uint16_t*, const uint16_t*) { return LM_EINVAL; }
int lm_upload_norm(lm_context*, int32_t, const float*) { return LM_EINVAL; }
int lm_upload_head(lm_context*, const float*, const uint16_t*, int64_t) { return LM_EINVAL; }
int lm_finalize_layer(lm_context*, int32_t) { return LM_EINVAL; }
}

namespace {

uint64_t g_state = 0;
long g_opened = 0, g_found = 0, g_read = 0;
uint64_t next() {  // splitmix64
    uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

std::vector<char> read_file(const char* path) {
    std::ifstream in(path, std::ios::binary);
    return std::vector<char>((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
}

const char* kFragments[] = {"{", "}", "[", "]", ",", ":", "\"", "\\", "\\u0000", "\\ud800", "-", "1e999",
                            "18446744073709551616", "-1", "0", "\"dtype\"", "\"shape\"", "\"data_offsets\"",
                            "\"BF16\"", "\"F32\"", "\"F16\"", "\"__metadata__\"", "null", "true", "[0,0]",
                            "[9223372036854775807]", "  ", "\n"};

void mutate(std::vector<char>& d) {
    const int n = 1 + static_cast<int>(next() % 4);
    for (int m = 0; m < n; ++m) {
        const uint64_t kind = next() % 6;
        if (kind == 0 && !d.empty()) {  // flip one bit
            d[next() % d.size()] ^= static_cast<char>(1u << (next() % 8));
        } else if (kind == 1 && !d.empty()) {  // set one byte
            d[next() % d.size()] = static_cast<char>(next() & 0xff);
        } else if (kind == 2 && !d.empty()) {  // truncate
            d.resize(next() % d.size());
        } else if (kind == 3) {  // insert a JSON fragment
            const char* f = kFragments[next() % (sizeof(kFragments) / sizeof(kFragments[0]))];
            const size_t at = d.empty() ? 0 : next() % d.size();
            d.insert(d.begin() + static_cast<std::ptrdiff_t>(at), f, f + std::strlen(f));
        } else if (kind == 4 && d.size() >= 8) {  // rewrite the 8-byte header length
            uint64_t len = 0;
            std::memcpy(&len, d.data(), 8);
            const uint64_t choice = next() % 4;
            len = choice == 0 ? len + (next() % 16) : choice == 1 ? len - (next() % 16) : choice == 2 ? next() : 0;
            std::memcpy(d.data(), &len, 8);
        } else if (kind == 5 && !d.empty()) {  // duplicate a span
            const size_t a = next() % d.size(), b = a + next() % (d.size() - a);
            const std::vector<char> span(d.begin() + static_cast<std::ptrdiff_t>(a), d.begin() + static_cast<std::ptrdiff_t>(b));
            d.insert(d.begin() + static_cast<std::ptrdiff_t>(next() % d.size()), span.begin(), span.end());
        }
    }
}

void exercise(const std::string& dir) {
    lm_checkpoint* ck = nullptr;
    if (lm_checkpoint_open(dir.c_str(), &ck) != LM_OK) {
        return;
    }
    ++g_opened;
    int64_t tensors = 0, shards = 0;
    (void)lm_checkpoint_count(ck, &tensors, &shards);
    for (const char* name : {"a", "b", "test.weight", "x", ""}) {
        int32_t dtype = 0, rank = 0;
        int64_t shape[8] = {};
        const void* payload = nullptr;
        uint64_t bytes = 0;
        if (lm_checkpoint_find(ck, name, &dtype, &rank, shape, &payload, &bytes) != LM_OK) {
            continue;
        }
        ++g_found;
        // touch the first and last payload bytes the reader hands out
        volatile char sink = 0;
        if (bytes > 0) {
            sink = static_cast<const char*>(payload)[0];
            sink = static_cast<const char*>(payload)[bytes - 1];
        }
        (void)sink;
        const void* p2 = nullptr;
        (void)lm_checkpoint_require(ck, name, rank, shape, dtype, &p2);
        uint64_t count = 1;
        for (int i = 0; i < rank; ++i) {
            count *= static_cast<uint64_t>(shape[i] > 0 ? shape[i] : 0);
        }
        if (count <= (1u << 20)) {
            std::vector<float> out(count + 1);
            if (lm_checkpoint_read_f32(ck, name, rank, shape, out.data(), count) == LM_OK) {
                ++g_read;
            }
        }
    }
    (void)lm_checkpoint_close(ck);
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 5) {
        std::fprintf(stderr, "usage: fuzz_checkpoint <work_dir> <iterations> <seed> <seed_file>...\n");
        return 2;
    }
    const std::string dir = argv[1];
    const long iterations = std::atol(argv[2]);
    g_state = std::strtoull(argv[3], nullptr, 10);
    std::vector<std::vector<char>> seeds;
    for (int i = 4; i < argc; ++i) {
        seeds.push_back(read_file(argv[i]));
    }
    const std::string path = dir + "/model.safetensors";
    for (long it = 0; it < iterations; ++it) {
        std::vector<char> d = seeds[next() % seeds.size()];
        if (it % 8 != 0) {  // keep some seeds unmutated
            mutate(d);
        }
        {
            std::ofstream out(path, std::ios::binary | std::ios::trunc);
            out.write(d.data(), static_cast<std::streamsize>(d.size()));
        }
        exercise(dir);
    }
    std::printf("fuzz_checkpoint: %ld cases (%ld opened, %ld tensors found, %ld read as f32), no fault\n", iterations,
                g_opened, g_found, g_read);
    return 0;
}
