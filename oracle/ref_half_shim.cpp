// ref_half_shim.cpp — exports the REFERENCE's own binary16 conversions
// (branes-ai/synapse, sdk/include/branes/synapse/numeric/half.hpp:18-82) with
// C linkage, so tests can compare oracle.cpp's restatement against them bit
// for bit. TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile straight
// from the header where it lies under /root/reference (it needs nothing but
// the standard library); the output goes to oracle/_ref/, never committed.
#include <branes/synapse/numeric/half.hpp>

#include <cstddef>
#include <cstdint>

extern "C" {
void ref_fp16_to_float_n(const std::uint16_t* h, float* out, std::size_t n) {
    for (std::size_t i = 0; i < n; ++i) {
        out[i] = branes::synapse::fp16_to_float(h[i]);
    }
}
void ref_float_to_fp16_n(const float* f, std::uint16_t* out, std::size_t n) {
    for (std::size_t i = 0; i < n; ++i) {
        out[i] = branes::synapse::float_to_fp16(f[i]);
    }
}
}
