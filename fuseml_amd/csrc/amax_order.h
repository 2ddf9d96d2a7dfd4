// amax_order.h — which 32-bit integer atomic carries a float maximum.
//
// Floats with the sign bit clear (+0.0 up to +inf, and the positive quiet NaN
// this code writes for every NaN) order like signed 32-bit integers; floats
// with the sign bit set (-0.0 down to -inf) order inversely like unsigned
// 32-bit integers.  A running maximum kept as the bits of a float (filled with
// -inf = 0xff800000) is therefore updated by
//   * a signed atomic max with the value's bits when its sign bit is clear,
//   * an unsigned atomic min with the value's bits when its sign bit is set.
// The dispatch is on the sign BIT, not on `v >= 0`: -0.0 compares equal to
// +0.0 but must take the unsigned path (as a signed int 0x80000000 is INT_MIN
// and would never beat the -inf fill or a stored negative value).
// A NaN is written as 0x7fc00000, which as a signed int exceeds every
// non-NaN float with the sign bit clear and as an unsigned int is below every
// float with the sign bit set, so the stored maximum stays NaN once any
// partial is NaN (torch.amax propagates NaN).
//
// Plain C++ with no HIP dependency: the kernel calls it on the device, and
// tests/test_amax_order.py compiles this same header on the host to check the
// dispatch against numpy's maximum over +-0, negatives, NaN and the -inf fill.
#pragma once

#include <stdint.h>

namespace fuseml_amax {

enum AtomicKind : int { kSignedMax = 0, kUnsignedMin = 1 };

// The atomic that folds the float with bits `vbits` into a running maximum,
// and the 32-bit operand to pass it.
__host__ __device__ inline AtomicKind atomic_for(uint32_t vbits, uint32_t* operand) {
  if ((vbits & 0x7fffffffu) > 0x7f800000u) {  // NaN, either sign
    *operand = 0x7fc00000u;
    return kSignedMax;
  }
  *operand = vbits;
  return (vbits >> 31) ? kUnsignedMin : kSignedMax;
}

}  // namespace fuseml_amax
