// check.h -- abort-on-error convention for the HIP backend (the reference's
// NOVA_CU / NOVA_REQUIRE, include/nova/memory/arena.h:276-289 and
// include/nova/config.h:47-63).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>

#define NOVA_HIP(call)                                                                   \
    do {                                                                                 \
        hipError_t nova_e_ = (call);                                                     \
        if (nova_e_ != hipSuccess) {                                                     \
            size_t nova_f_ = 0, nova_t_ = 0;                                             \
            (void)hipMemGetInfo(&nova_f_, &nova_t_);                                     \
            std::fflush(stdout);                                                         \
            std::fprintf(stderr, "[nova] FATAL %s:%d %s -> %s (free %.2f / total %.2f GiB)\n", \
                         __FILE__, __LINE__, #call, hipGetErrorString(nova_e_),          \
                         nova_f_ / 1073741824.0, nova_t_ / 1073741824.0);                \
            std::fflush(stderr);                                                         \
            std::abort();                                                                \
        }                                                                                \
    } while (0)

#define NOVA_REQUIRE(cond)                                                               \
    do {                                                                                 \
        if (!(cond)) {                                                                   \
            std::fflush(stdout);                                                         \
            std::fprintf(stderr, "[nova] FATAL %s:%d requirement failed: %s\n", __FILE__,  \
                         __LINE__, #cond);                                               \
            std::fflush(stderr);                                                         \
            std::abort();                                                                \
        }                                                                                \
    } while (0)

// launch-error check after every launch (the reference checks at op end, model.h:56-60)
#define NOVA_LAUNCHED() NOVA_HIP(hipGetLastError())
