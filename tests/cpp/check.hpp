// Minimal test harness for the C++ host tests: CHECK records a failure and
// carries on; main() returns the failure count.
#pragma once

#include <cstdio>

namespace check {
inline int failures = 0;
inline int checks = 0;
}  // namespace check

#define CHECK(cond)                                                              \
    do {                                                                         \
        ++check::checks;                                                         \
        if (!(cond)) {                                                           \
            ++check::failures;                                                   \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
        }                                                                        \
    } while (0)

#define CHECK_DONE()                                                                       \
    do {                                                                                   \
        std::printf("%d checks, %d failures\n", check::checks, check::failures);          \
        return check::failures == 0 ? 0 : 1;                                               \
    } while (0)
