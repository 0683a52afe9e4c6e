// The range of values the fixed-point accumulators take, free of HIP so that host tests compile
// it too.  A check here is false for NaN and for both infinities (every comparison with NaN is
// false, and |inf| is not below any bound).
#pragma once
#if defined(__HIPCC__)
#define Q35_FX_HD __host__ __device__
#else
#define Q35_FX_HD
#endif

namespace q35 {

// A contribution to a plain fixed-point word (value * 2^32 in a signed 64-bit integer): finite
// and |v| < 2^31, so that v * 2^32 rounds to an integer inside (-2^63, 2^63).
Q35_FX_HD inline bool fx_addable(float v) { return __builtin_fabsf(v) < 2147483648.0f; }

// A contribution to a counted word of the persistent step kernel (value * 2^32 plus an 8-bit
// contribution count in the top byte): |v| < 2^22, so that a word's total, at most a few hundred
// such values of either sign in practice and |total| < 2^23 by contract, stays inside the 55-bit
// value field.
Q35_FX_HD inline bool fxc_addable(float v) { return __builtin_fabsf(v) < 4194304.0f; }

}  // namespace q35
