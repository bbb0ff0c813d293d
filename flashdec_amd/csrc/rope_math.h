// Split-half RoPE arithmetic shared by the RoPE + append kernel and the
// decode kernel's fused RoPE, so that both produce the same bits.
//
// Reference: flashdec/rope.py:26-85 (apply_rope).  Frequency i of a rotary
// width R is inv = base^(-2i / R) with the exponent formed in fp32 as torch
// forms -arange(0, R, 2) / R; the angle is fp32(pos) * inv in fp32.  The two
// transcendental steps -- base^e and cos/sin(angle) -- are evaluated in
// float64 and rounded once to fp32, i.e. the correctly rounded values of the
// reference's fp32 expressions.  The rotation of a pair (x1, x2) is
//   lo = rn(rn(x1 * c) - rn(x2 * s)),  hi = rn(rn(x2 * c) + rn(x1 * s))
// with contraction into FMAs switched off, then rounded to the element type.
//
// Table mode: the caller passes cos/sin already evaluated (e.g. by the
// reference's own torch expression on the same device, flashdec/rope.py:
// 66-70), and only the rotation above runs here, so the result equals that
// expression's rotation bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace fd {

__device__ __forceinline__ void rope_cos_sin(float base, int rotary_dim, int64_t pos, int i, float& c, float& s) {
  const float e = static_cast<float>(-2 * i) / static_cast<float>(rotary_dim);
  const float inv = static_cast<float>(pow(static_cast<double>(base), static_cast<double>(e)));
  const float ang = static_cast<float>(pos) * inv;
  double sd, cd;
  sincos(static_cast<double>(ang), &sd, &cd);
  c = static_cast<float>(cd);
  s = static_cast<float>(sd);
}

// cos/sin of frequency i at position pos from a caller-built fp32 table
// [2, rows, half] (plane 0 cos, plane 1 sin, row = position).  Positions
// outside [0, rows) read the nearest row, which keeps the loads in bounds;
// callers keep positions below rows (the checked Python entry points
// verify it).
__device__ __forceinline__ void rope_table_cos_sin(const float* tab, int64_t rows, int half, int64_t pos, int i,
                                                   float& c, float& s) {
  const int64_t r = pos < 0 ? 0 : (pos < rows ? pos : rows - 1);
  c = tab[r * half + i];
  s = tab[(rows + r) * half + i];
}

__device__ __forceinline__ void rope_rotate(float x1, float x2, float c, float s, float& lo, float& hi) {
#pragma clang fp contract(off)
  const float t0 = x1 * c;
  const float t1 = x2 * s;
  const float t2 = x2 * c;
  const float t3 = x1 * s;
  lo = t0 - t1;
  hi = t2 + t3;
}

}  // namespace fd
