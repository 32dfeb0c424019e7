// Device side of CopyLaunch: block b of the launch's copy blocks moves blockDim.x 8-channel
// groups (16 bytes each, aligned: the loader keeps every view offset, width and row stride a
// multiple of 8 halves) of the copy whose block range holds b.  Shared by k_copyc and the
// attention kernel, which carries copies in its trailing blocks.
#pragma once
#include "engine.hpp"

namespace yolo {

__device__ __forceinline__ void runCopyBlock(const CopyLaunch& L, int b) {
  typedef f16 f16x8c __attribute__((ext_vector_type(8)));
  int pj = 0;
#pragma unroll
  for (int q = 1; q < COPY_GROUP; q++)
    if (q < L.n && b >= L.blk0[q]) pj = q;
  pj = __builtin_amdgcn_readfirstlane(pj);
  const View x = L.x[pj], y = L.y[pj];
  const int idx = (b - L.blk0[pj]) * (int)blockDim.x + (int)threadIdx.x;
  if (idx >= L.total[pj]) return;
  const int cg = y.C >> 3, g = idx % cg;
  const size_t m = idx / cg;
  *(f16x8c*)(y.p + m * y.s + y.o + g * 8) = *(const f16x8c*)(x.p + m * x.s + x.o + g * 8);
}

}  // namespace yolo
