// Device helpers shared by the decode and NMS kernels: the packed candidate key and the
// axis-aligned suppression test.  Every file that includes this is built with
// -ffp-contract=off, so the fp32 expressions round exactly as written.
#pragma once
#include "engine.hpp"

namespace yolo {

// Candidate key: score bits in the high word, 0xFFFFFFFF - anchor in the low word, so one
// unsigned compare orders candidates by (score desc, anchor asc) -- the reference's rank
// order with ties broken by anchor index.
__device__ __forceinline__ unsigned long long packKey(float score, int anchor) {
  return ((unsigned long long)__float_as_uint(score) << 32) | (unsigned)(0xFFFFFFFFu - (unsigned)anchor);
}

__device__ __forceinline__ int keyAnchor(unsigned long long k) {
  return (int)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFull));
}

// A value every lane of the wave holds (an LDS word read at a uniform address), moved to a
// scalar register so the control flow that depends on it stays scalar.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// (compare-selects rather than fmaxf/fminf: box coordinates are finite, and the selects need
// no NaN canonicalisation of their operands)
__device__ __forceinline__ float fmx(float a, float b) { return a > b ? a : b; }
__device__ __forceinline__ float fmn(float a, float b) { return a < b ? a : b; }

// Box a (the higher-ranked, kept candidate) suppresses box b iff inter/union > thr, with a
// union > 0 guard (engine/engine.cu:1091-1109: areas and union in that order of operations).
// Decided without the division unless the two sides are within a few ulps; then the
// division decides, exactly as the reference writes it.
__device__ __forceinline__ bool suppresses(float4 a, float4 b, float thr) {
  const float xx1 = fmx(a.x, b.x), yy1 = fmx(a.y, b.y);
  const float xx2 = fmn(a.z, b.z), yy2 = fmn(a.w, b.w);
  const float w = fmx(0.f, xx2 - xx1), h = fmx(0.f, yy2 - yy1);
  const float inter = w * h;
  const float aarea = (a.z - a.x) * (a.w - a.y);
  const float barea = (b.z - b.x) * (b.w - b.y);
  const float ua = aarea + barea - inter;
  if (!(ua > 0.f)) return false;
  const float p = thr * ua;
  if (inter > p * 1.000001f) return true;
  if (inter < p * 0.999999f) return false;
  return inter / ua > thr;
}

// probiou of two rotated boxes as Gaussians (centre x, y; covariance [[A, C], [C, B]];
// det = max(A*B - C*C, 0)): the ultralytics batch_probiou expression that k_nms_obb
// evaluates (engine/engine.cu:1160-1176), eps 1e-7 in the t1/t2 denominator, in the t3
// sqrt denominator and added to the log argument, bd clamped to [eps, 100].
__device__ __forceinline__ float probiou(float2 p1, float4 g1, float det1, float2 p2, float4 g2,
                                         float det2) {
  const float eps = 1e-7f;
  const float dx = p1.x - p2.x, dy = p1.y - p2.y;
  const float sA = g1.x + g2.x, sB = g1.y + g2.y, sC = g1.z + g2.z;
  const float disc = sA * sB - sC * sC;
  const float den = disc + eps;
  const float t1 = 0.25f * (sA * dy * dy + sB * dx * dx) / den;
  const float t2 = 0.5f * (sC * (-dx) * dy) / den;
  const float t3 = 0.5f * logf(disc / (4.f * sqrtf(det1 * det2) + eps) + eps);
  const float bd = fminf(fmaxf(t1 + t2 + t3, eps), 100.f);
  return 1.f - sqrtf(1.f - expf(-bd) + eps);
}

// The far-pair bound of the rotated NMS: for covariances with determinant >= OBB_DET_MIN and
// condition number below ~1e4 (det >= OBB_COND * trace^2), bd >= |d|^2 / (4 trace(S1 + S2)),
// and probiou >= thr needs bd <= B* = -ln(1 + eps - (1 - thr)^2), so |d|^2 > 8 B* trace
// (a factor-2 margin over fp32 rounding) rules a pair out; used for 0.05 <= thr <= 0.95.
constexpr float OBB_DET_MIN = 1.f;
constexpr float OBB_COND = 1e-4f;

}  // namespace yolo
