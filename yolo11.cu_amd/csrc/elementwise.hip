// Bandwidth-bound NHWC view kernels: ADD, MAXPOOL5, UPSAMPLE2, COPYC, PS2.
// Each thread moves one 8-channel group (16 bytes) of one pixel; the loader guarantees
// every view offset, width and row stride is a multiple of 8 halves, so all accesses
// are aligned 128-bit loads/stores.  Semantics follow the reference ops
// (engine/engine.cu:663-732; torch definitions export/export.py:475-491).
#include "engine.hpp"

namespace yolo {

typedef f16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f16x8 ld8(const View& v, size_t pix, int c) {
  return *(const f16x8*)(v.p + pix * v.s + v.o + c);
}
__device__ __forceinline__ void st8(const View& v, size_t pix, int c, f16x8 x) {
  *(f16x8*)(v.p + pix * v.s + v.o + c) = x;
}

__global__ __launch_bounds__(256) void k_add(View a, View b, View y, int total) {
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  int cg = y.C >> 3, g = idx % cg;
  size_t m = idx / cg;
  f16x8 va = ld8(a, m, g * 8), vb = ld8(b, m, g * 8), o;
#pragma unroll
  for (int j = 0; j < 8; j++) o[j] = (f16)((float)va[j] + (float)vb[j]);
  st8(y, m, g * 8, o);
}

// 5x5 stride-1 max pool with implicit -inf padding of 2 (F.max_pool2d(x, 5, 1, 2)).
__global__ __launch_bounds__(256) void k_maxpool5(View x, View y, int total) {
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  int cg = y.C >> 3, g = idx % cg, m = idx / cg;
  int HW = y.H * y.W, img = m / HW, rem = m - img * HW;
  int oy = rem / y.W, ox = rem - oy * y.W;
  f16x8 mx;
#pragma unroll
  for (int j = 0; j < 8; j++) mx[j] = (f16)(-65504.0f);
  for (int dy = -2; dy <= 2; dy++) {
    int iy = oy + dy;
    if (iy < 0 || iy >= x.H) continue;
    for (int dx = -2; dx <= 2; dx++) {
      int ix = ox + dx;
      if (ix < 0 || ix >= x.W) continue;
      f16x8 v = ld8(x, (size_t)(img * x.H + iy) * x.W + ix, g * 8);
#pragma unroll
      for (int j = 0; j < 8; j++) mx[j] = v[j] > mx[j] ? v[j] : mx[j];
    }
  }
  st8(y, m, g * 8, mx);
}

// nearest x2: out(oy, ox) = in(oy/2, ox/2)
__global__ __launch_bounds__(256) void k_upsample2(View x, View y, int total) {
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  int cg = y.C >> 3, g = idx % cg, m = idx / cg;
  int HW = y.H * y.W, img = m / HW, rem = m - img * HW;
  int oy = rem / y.W, ox = rem - oy * y.W;
  st8(y, m, g * 8, ld8(x, (size_t)(img * x.H + (oy >> 1)) * x.W + (ox >> 1), g * 8));
}

__global__ __launch_bounds__(256) void k_copyc(View x, View y, int total) {
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  int cg = y.C >> 3, g = idx % cg;
  size_t m = idx / cg;
  st8(y, m, g * 8, ld8(x, m, g * 8));
}

// pixel shuffle r=2 from quadrant-major channel blocks: in(i, j, q*C + c) -> out(2i+di, 2j+dj, c)
// with q = 2*di + dj.  After a 1x1 conv to 4C this is ConvTranspose2d(k=2, s=2) exactly.
__global__ __launch_bounds__(256) void k_ps2(View x, View y, int total) {
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  int cg = y.C >> 3, g = idx % cg, m = idx / cg;
  int HW = y.H * y.W, img = m / HW, rem = m - img * HW;
  int oy = rem / y.W, ox = rem - oy * y.W;
  int q = ((oy & 1) << 1) | (ox & 1);
  st8(y, m, g * 8, ld8(x, (size_t)(img * x.H + (oy >> 1)) * x.W + (ox >> 1), q * y.C + g * 8));
}

static inline int grid(int total) { return (total + 255) / 256; }

void launchAdd(const View& a, const View& b, const View& y, int Bn, hipStream_t st) {
  int total = Bn * y.H * y.W * (y.C / 8);
  k_add<<<grid(total), 256, 0, st>>>(a, b, y, total);
}
void launchMaxPool5(const View& x, const View& y, int Bn, hipStream_t st) {
  int total = Bn * y.H * y.W * (y.C / 8);
  k_maxpool5<<<grid(total), 256, 0, st>>>(x, y, total);
}
void launchUpsample2(const View& x, const View& y, int Bn, hipStream_t st) {
  int total = Bn * y.H * y.W * (y.C / 8);
  k_upsample2<<<grid(total), 256, 0, st>>>(x, y, total);
}
void launchCopyC(const View& x, const View& y, int Bn, hipStream_t st) {
  int total = Bn * y.H * y.W * (y.C / 8);
  k_copyc<<<grid(total), 256, 0, st>>>(x, y, total);
}
void launchPS2(const View& x, const View& y, int Bn, hipStream_t st) {
  int total = Bn * y.H * y.W * (y.C / 8);
  k_ps2<<<grid(total), 256, 0, st>>>(x, y, total);
}

}  // namespace yolo
