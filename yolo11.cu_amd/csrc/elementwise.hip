// Bandwidth-bound NHWC view kernels: ADD, MAXPOOL5 (and the fused SPPF pool chain),\n// UPSAMPLE2, COPYC, PS2.
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
// Window taps are clamped to the image instead of skipped: a clamped tap lands on a border
// pixel that is inside the window anyway, so the max is unchanged, and the 25 loads carry
// no branches and can all be in flight together.
__global__ __launch_bounds__(256) void k_maxpool5(View x, View y, int total) {
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  int cg = y.C >> 3, g = idx % cg, m = idx / cg;
  int HW = y.H * y.W, img = m / HW, rem = m - img * HW;
  int oy = rem / y.W, ox = rem - oy * y.W;
  f16x8 v[25];
#pragma unroll
  for (int dy = 0; dy < 5; dy++) {
    const int iy = min(max(oy + dy - 2, 0), x.H - 1);
#pragma unroll
    for (int dx = 0; dx < 5; dx++) {
      const int ix = min(max(ox + dx - 2, 0), x.W - 1);
      v[dy * 5 + dx] = ld8(x, (size_t)(img * x.H + iy) * x.W + ix, g * 8);
    }
  }
  f16x8 mx = v[0];
#pragma unroll
  for (int t = 1; t < 25; t++)
#pragma unroll
    for (int j = 0; j < 8; j++) mx[j] = v[t][j] > mx[j] ? v[t][j] : mx[j];
  st8(y, m, g * 8, mx);
}

// SPPF pool chain: y1 = mp5(x), y2 = mp5(y1), y3 = mp5(y2) in one launch (the reference
// runs three MAXPOOL5 ops, export/export.py:475-491).  With windows clipped at the border,
// mp5(mp5(x)) is the clipped 9-wide max of x and mp5 applied three times the clipped 13-wide
// max, so the three outputs are separable 5-, 9- and 13-wide maxima of x: one row pass
// (planes r5, r9, r13 from one growing window) and one column pass, with the x plane of one
// (image, 8-channel group) per block in LDS.  Max is exact, so this equals the chained pools.
__device__ __forceinline__ f16x8 max8(f16x8 a, f16x8 b) { return __builtin_elementwise_max(a, b); }

__global__ __launch_bounds__(256) void k_sppf_pool(View x, View y1, View y2, View y3) {
  extern __shared__ f16x8 sp[];
  const int H = x.H, W = x.W, HW = H * W;
  f16x8* a = sp;
  f16x8* r5 = sp + HW;
  f16x8* r9 = r5 + HW;
  f16x8* r13 = r9 + HW;
  const int g = blockIdx.x, img = blockIdx.y;
  const size_t pix0 = (size_t)img * HW;
  for (int p0 = 0; p0 < HW; p0 += 4 * 256) {   // 4 loads in flight per thread
    f16x8 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int p = p0 + u * 256 + threadIdx.x;
      if (p < HW) v[u] = ld8(x, pix0 + p, g * 8);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int p = p0 + u * 256 + threadIdx.x;
      if (p < HW) a[p] = v[u];
    }
  }
  __syncthreads();
  for (int p = threadIdx.x; p < HW; p += blockDim.x) {
    const int py = p / W, px = p - py * W;
    const f16x8* row = a + py * W;
    f16x8 m = row[px];
#pragma unroll
    for (int d = 1; d <= 6; d++) {
      if (px >= d) m = max8(m, row[px - d]);
      if (px + d < W) m = max8(m, row[px + d]);
      if (d == 2) r5[p] = m;
      if (d == 4) r9[p] = m;
    }
    r13[p] = m;
  }
  __syncthreads();
  for (int p = threadIdx.x; p < HW; p += blockDim.x) {
    const int py = p / W;
    f16x8 m5 = r5[p], m9 = r9[p], m13 = r13[p];
#pragma unroll
    for (int d = 1; d <= 6; d++) {
      if (py >= d) {
        if (d <= 2) m5 = max8(m5, r5[p - d * W]);
        if (d <= 4) m9 = max8(m9, r9[p - d * W]);
        m13 = max8(m13, r13[p - d * W]);
      }
      if (py + d < H) {
        if (d <= 2) m5 = max8(m5, r5[p + d * W]);
        if (d <= 4) m9 = max8(m9, r9[p + d * W]);
        m13 = max8(m13, r13[p + d * W]);
      }
    }
    st8(y1, pix0 + p, g * 8, m5);
    st8(y2, pix0 + p, g * 8, m9);
    st8(y3, pix0 + p, g * 8, m13);
  }
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
size_t sppfPoolLds(int H, int W) { return (size_t)4 * H * W * sizeof(f16x8); }
void launchSppfPool(const View& x, const View& y1, const View& y2, const View& y3, int Bn,
                    hipStream_t st) {
  k_sppf_pool<<<dim3(x.C / 8, Bn), 256, sppfPoolLds(x.H, x.W), st>>>(x, y1, y2, y3);
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
