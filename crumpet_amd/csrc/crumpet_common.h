// Shared helpers of the gfx950 shifted-window kernels.
//
// Host and device code both include this header; the FastDiv part also
// compiles with a plain C++ compiler so the CPU tests can check it.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define CRUMPET_HD __host__ __device__ __forceinline__
#else
#define CRUMPET_HD inline
#endif

namespace crumpet {

// Division of a non-negative 31-bit numerator by a run-time invariant
// divisor d in [1, 2^31) with one multiply-high, one add and one shift.
//
// Method: Granlund & Montgomery, "Division by invariant integers using
// multiplication" (PLDI 1994), Theorem 4.2 with N = 32.  With
// l = ceil(log2 d) and m' = floor(2^32 (2^l - d) / d) + 1, the quotient is
// floor((m' + 2^32) n / 2^(32+l)) = (mulhi(m', n) + n) >> l.  Restricting
// n < 2^31 keeps mulhi(m', n) + n below 2^32, so the sum needs no carry
// handling.
struct FastDiv {
    uint32_t d;
    uint32_t m;
    uint32_t l;

    FastDiv() : d(1), m(1), l(0) {}
    explicit FastDiv(uint32_t divisor) { init(divisor); }

    void init(uint32_t divisor) {
        d = divisor;
        uint32_t lg = 0;
        while (lg < 32 && (uint64_t(1) << lg) < divisor) ++lg;
        l = lg;
        const uint64_t num = ((uint64_t(1) << lg) - divisor) << 32;
        m = static_cast<uint32_t>(num / divisor + 1);
    }

    CRUMPET_HD uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
        const uint32_t t = __umulhi(m, n);
#else
        const uint32_t t = static_cast<uint32_t>((uint64_t(m) * n) >> 32);
#endif
        return (t + n) >> l;
    }

    CRUMPET_HD void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
        q = div(n);
        r = n - q * d;
    }
};

}  // namespace crumpet

#if defined(__HIPCC__)

namespace crumpet {

// Number of XCDs (accelerator complex dies) of MI355X; consecutive
// workgroup ids are dispatched round-robin over them.
constexpr uint32_t kNumXcd = 8;

// Remap the hardware workgroup id so that each XCD receives one contiguous
// range of logical work chunks (neighbouring chunks then share an L2).
// `launched` must be a multiple of kNumXcd; ids that map past `chunks`
// return false and the workgroup has no work.
__device__ __forceinline__ bool xcd_chunk(uint32_t hw_id, uint32_t launched,
                                          uint32_t chunks, uint32_t& chunk) {
    const uint32_t per_xcd = launched / kNumXcd;
    chunk = (hw_id % kNumXcd) * per_xcd + hw_id / kNumXcd;
    return chunk < chunks;
}

inline uint32_t xcd_launch_count(uint32_t chunks) {
    return (chunks + kNumXcd - 1) / kNumXcd * kNumXcd;
}

}  // namespace crumpet

// Error bookkeeping shared by every C-ABI entry point.
namespace crumpet {
void set_last_error(const char* fmt, ...);
int fail(int status, const char* fmt, ...);
int check_launch(const char* what);
}  // namespace crumpet

#endif  // __HIPCC__
