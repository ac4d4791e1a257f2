// Shared host-side plumbing of the C ABI: status + last-error, launch counters,
// argument checks.  Device code does not include this file's helpers.
#pragma once

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/rwkv_hip.h"

namespace rwkv {

// Thread-local message behind rwkv_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

struct Counters {
    std::atomic<int64_t> seq_fwd{0}, chunk_fwd{0}, train_fwd{0}, train_bwd{0}, step{0}, tail{0},
        sb6_dequant{0}, sym_dequant{0}, sb6_gemv{0}, sym_gemv{0}, sym_fused{0}, step_tail{0}, sb6_fused{0}, sym_rows{0}, x070{0}, sb6_gemm{0}, seq_chunked{0}, sb6_batch{0},
        sym_gemm{0};
};
Counters& counters();

// Events armed by rwkv_time_next_launch() for the calling thread; taking them
// disarms the hook.
struct TimingEvents {
    void* start;
    void* stop;
};
TimingEvents take_timing();

inline bool dtype_ok(int dt) { return dt == RWKV_F32 || dt == RWKV_BF16 || dt == RWKV_F16; }
inline int64_t dtype_size(int dt) { return dt == RWKV_F32 ? 4 : 2; }

}  // namespace rwkv

#define RWKV_REQUIRE(cond, status, ...)          \
    do {                                         \
        if (!(cond)) {                           \
            ::rwkv::set_error(__VA_ARGS__);      \
            return (status);                     \
        }                                        \
    } while (0)
