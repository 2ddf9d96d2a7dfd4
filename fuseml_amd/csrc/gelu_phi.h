// gelu_phi.h — the normal CDF behind GELU (approximate='none'), shared by the
// GEMM+epilogue kernels and the single-kernel MLP block.
//
//   Phi(x) = 0.5 (1 + erf(x / sqrt 2)) ~= 0.5 + xc * Q(xc^2),
//   xc = clamp(x, +-3 sqrt 2).
//
// Q is the least-squares fit of erf(z)/z in z^2 on [0, 3] under the constraint
// that the fit reaches erf's limit at the clamp (fit_erf.py in this directory
// prints these constants), with the 1/sqrt 2 and 1/2 scalings folded in:
// Q_k = P_k / (2 sqrt 2 * 2^k); Q_0 is moved by a few ulps so that the float32
// evaluation gives Phi = 1 at +3 sqrt 2 and Phi = 2e-8 at -3 sqrt 2.  So
// GELU(x) = x Phi(xc) is x beyond the clamp and ~0 below it.  |Phi error| <=
// 1.5e-5 in float32.  Only FMAs: GELU costs 12 VALU ops and no quarter-rate
// transcendentals.
#ifndef FUSEML_GELU_PHI_H_
#define FUSEML_GELU_PHI_H_

namespace fuseml_phi {
constexpr float kPhiClamp = 4.2426406871192851f;  // 3 sqrt 2
constexpr float kPhiQ0 = 3.989046812e-01f;
constexpr float kPhiQ1 = -6.635335088e-02f;
constexpr float kPhiQ2 = 9.824221022e-03f;
constexpr float kPhiQ3 = -1.111894497e-03f;
constexpr float kPhiQ4 = 9.411587962e-05f;
constexpr float kPhiQ5 = -5.707656783e-06f;
constexpr float kPhiQ6 = 2.308580349e-07f;
constexpr float kPhiQ7 = -5.510266465e-09f;
constexpr float kPhiQ8 = 5.820578394e-11f;
}  // namespace fuseml_phi

#endif  // FUSEML_GELU_PHI_H_
