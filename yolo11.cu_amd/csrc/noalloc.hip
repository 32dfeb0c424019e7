// Decode + NMS of caller-provided detect heads with no device allocation: the candidate
// records, the per-image candidate lists and counters, the survivors' anchor indices and the
// post-processing parameters live in one file-scope device array (`scratch`) of fixed size,
// so the entry point can run where hipMalloc cannot (inside a stream capture, in serving
// loops that forbid allocation).  The kernels are the engine's own decode and NMS kernels.
//
// Every call on a GPU uses that GPU's one copy of the array, and the array keeps the last
// call's contents: calls that overlap on one GPU (two streams, two host threads) race.
#include <mutex>

#include "engine.hpp"

#include "../../include/yolo.h"

namespace yolo {
namespace {

constexpr size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

constexpr int kMaxBatch = YOLO_STATIC_MAX_BATCH;
constexpr size_t kMaxSlots = YOLO_STATIC_MAX_ANCHOR_SLOTS;   // images x anchors
constexpr int kCandStride = 6;                                // x1 y1 x2 y2 score cls

// byte offsets of the regions inside the array
constexpr size_t kParamsOff = 0;                                            // PostParams
constexpr size_t kCountsOff = 256;                                          // int [kMaxBatch]
constexpr size_t kRawOff = kCountsOff + align256(kMaxBatch * sizeof(int));  // int [kMaxBatch]
constexpr size_t kIdxOff = kRawOff + align256(kMaxBatch * sizeof(int));     // int [kMaxBatch][MAX_OUT]
constexpr size_t kListOff = kIdxOff + align256((size_t)kMaxBatch * MAX_OUT * sizeof(int));
constexpr size_t kCandOff = kListOff + align256(kMaxSlots * sizeof(unsigned long long));
constexpr size_t kScratchBytes = kCandOff + align256(kMaxSlots * kCandStride * sizeof(float));
static_assert(sizeof(PostParams) <= 256, "params region");

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// Host-side device address of `scratch`, per device: the array's name in host code is only a
// stand-in, so the address comes from hipGetSymbolAddress with that device current.
constexpr int kMaxDevices = 64;
std::mutex gMu;
unsigned char* gScratch[kMaxDevices] = {};

unsigned char* scratchPtr(std::string& err) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    err = "no current HIP device";
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(gMu);
  if (!gScratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      err = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e);
      return nullptr;
    }
    gScratch[dev] = static_cast<unsigned char*>(p);
  }
  return gScratch[dev];
}

// Writes the post-processing parameters and zeroes the per-image candidate counters (the
// decode kernel appends to them; a fill kernel rather than a memset node keeps the call
// capturable).
__global__ void k_static_init(PostParams* prm, int* counts, int Bn, float conf, float iou, int max_det) {
  const int t = threadIdx.x;
  if (t == 0) *prm = PostParams{conf, iou, max_det, 0};
  for (int i = t; i < Bn; i += blockDim.x) counts[i] = 0;
}

bool viewOk(const void* p, int stride, int off, int C, std::string& err, const char* what) {
  if (!p) { err = std::string(what) + " pointer is NULL"; return false; }
  if (((uintptr_t)p & 15) || stride % 8 || off % 8 || stride < off + C) {
    err = std::string(what) + " view must be 16-byte aligned with stride and offset multiples of 8 "
          "halves and hold the channels it is read at";
    return false;
  }
  return true;
}

}  // namespace
}  // namespace yolo

extern "C" int yolo_detect_static(const YoloHeadLevel* levels, int nlev, int B, int nc, float conf, float iou,
                                  int max_det, float* dets, int* counts, int* raw_counts, hipStream_t stream) {
  using namespace yolo;
  std::string err;
  auto fail = [&](const std::string& m) {
    fprintf(stderr, "yolo_detect_static: %s\n", m.c_str());
    return -1;
  };
  if (!levels || nlev < 1 || nlev > 3) return fail("nlev must be 1..3");
  if (B < 1 || B > kMaxBatch) return fail("B must be 1.." + std::to_string(kMaxBatch));
  if (nc < 1 || nc > 1024) return fail("nc must be 1..1024");
  if (!(conf >= 0.f) || !(iou >= 0.f) || max_det < 0 || max_det > MAX_OUT)
    return fail("conf and iou must be >= 0 and max_det 0..300");
  if (!dets || !counts) return fail("dets and counts must be device pointers");
  const int ncpad = (nc + 7) / 8 * 8;
  DecodeArgs a{};
  long A = 0;
  for (int l = 0; l < nlev; l++) {
    const YoloHeadLevel& L = levels[l];
    if (L.H < 1 || L.W < 1 || L.stride < 1) return fail("level " + std::to_string(l) + ": bad H, W or stride");
    if (!viewOk(L.box, L.box_stride, L.box_off, 64, err, "box") ||
        !viewOk(L.cls, L.cls_stride, L.cls_off, ncpad, err, "cls"))
      return fail("level " + std::to_string(l) + ": " + err);
    DecodeLevel& D = a.lv[l];
    D.box = View{(f16*)L.box, L.H, L.W, L.box_stride, L.box_off, 64};
    D.cls = View{(f16*)L.cls, L.H, L.W, L.cls_stride, L.cls_off, ncpad};
    D.coef = View{nullptr, 0, 0, 0, 0, 0};
    D.H = L.H;
    D.W = L.W;
    D.stride = L.stride;
    D.base = (int)A;
    A += (long)L.H * L.W;
  }
  if ((size_t)A * B > kMaxSlots)
    return fail("B x anchors = " + std::to_string((size_t)A * B) + " exceeds the static maximum " +
                std::to_string(kMaxSlots));
  a.nlev = nlev;
  a.A = (int)A;
  a.nc = nc;
  a.nm = 0;
  a.obb = 0;
  unsigned char* s = scratchPtr(err);
  if (!s) return fail(err);
  PostParams* prm = reinterpret_cast<PostParams*>(s + kParamsOff);
  int* cnt = reinterpret_cast<int*>(s + kCountsOff);
  int* raw = raw_counts ? raw_counts : reinterpret_cast<int*>(s + kRawOff);
  int* outidx = reinterpret_cast<int*>(s + kIdxOff);
  unsigned long long* lists = reinterpret_cast<unsigned long long*>(s + kListOff);
  float* cand = reinterpret_cast<float*>(s + kCandOff);
  k_static_init<<<1, 64, 0, stream>>>(prm, cnt, B, conf, iou, max_det);
  launchDecode(a, cand, lists, cnt, prm, B, stream);
  launchNms(cand, lists, cnt, (int)A, kCandStride, dets, outidx, counts, raw, prm, B, stream);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(std::string("launch failed: ") + hipGetErrorString(e));
  return 0;
}
