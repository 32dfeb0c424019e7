// Host runtime of the MI355X YOLO engine and its C ABI (include/yolo.h).
//
// Mirrors the reference's host side (engine/engine.cu): loadGraph (:88-248), runOp
// (:1261-1453), forward (:1455-1481), fuseAdds (:1484-1501), autotune (:1503-1533),
// per-B graph capture and calibration (:1665-1695) and the embedding API (:1653-1794),
// plus the CLI's dump / pipeline / profile / bench modes (:1843-2090) as C entry points.
//
// Memory layout in HBM: every activation buffer of the graph is an NHWC fp16 region of
// B_max images carved from one arena (256-byte aligned); a tensor is a channel slice of a
// buffer, so split/concat cost nothing.  Candidates use one fixed slot per anchor
// ([B][A][6 + nm] fp32) plus a key array ([B][A] fp32), so decode needs no counter reset
// and no atomics, and every graph replay starts from a clean state.
#include "engine.hpp"
#include "jpeg.hpp"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <tuple>
#include <condition_variable>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/yolo.h"

namespace yolo {

struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};

static std::string fmt(const char* f, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

#define HCK(x)                                                                                    \
  do {                                                                                            \
    hipError_t e_ = (x);                                                                          \
    if (e_ != hipSuccess)                                                                         \
      throw yolo::Failure(yolo::fmt("HIP error %s at %s:%d", hipGetErrorString(e_), __FILE__, __LINE__)); \
  } while (0)

struct SlotGeom {
  float scale = 1.f;
  int top = 0, left = 0;
};

// Classify geometry (torchvision Resize(S) + CenterCrop(S), engine/engine.cu:1036-1046):
// the shortest edge becomes S and the long edge S * long / short (integer truncation); the
// crop offsets round half to even, as Python's round() does.
struct ClsGeom {
  int rh, rw, top, left;
};
static ClsGeom clsGeom(int S, int sh, int sw) {
  const long rh = sw <= sh ? (long)S * sh / sw : S;
  const long rw = sw <= sh ? S : (long)S * sw / sh;
  auto half = [](long d) { return (int)(d / 2 + ((d & 1) && ((d / 2) & 1) ? 1 : 0)); };
  return ClsGeom{(int)rh, (int)rw, half(rh - S), half(rw - S)};
}

struct Engine {
  GraphDesc g;
  std::vector<OpDesc> ops;
  int B = 1;
  hipStream_t st = nullptr;
  // device memory
  void* arena = nullptr;
  std::vector<f16*> bufp;
  f16* weights = nullptr;
  float* bias = nullptr;
  size_t nweights = 0, nbias = 0;
  float* cand = nullptr;
  int* nmsCount = nullptr;            // per-image decode list length (NMS re-arms it)
  unsigned long long* nmsScratch = nullptr;
  NmsImage* nmsWork = nullptr;        // multi-block NMS workspace, one record per image
  bool nmsBlock = false;              // YOLO_NMS_BLOCK: one-block NMS (no workspace)
  // results: [outcnt B][rawcnt B] then (256-aligned) outdets B*MAX_OUT*outK in one block, so
  // one copy brings everything the host reads back
  void* results = nullptr;
  size_t detOff = 0;
  float* outdets = nullptr;
  int* outidx = nullptr;
  int* outcnt = nullptr;
  int* rawcnt = nullptr;
  uint8_t* masks = nullptr;
  PostParams* params = nullptr;
  // split-K partial tiles and tile counters: per-op regions (wsOff / cntOff) after tuning
  float* splitWs = nullptr;
  int* splitCnt = nullptr;
  size_t splitWsBytes = 0, splitCntN = 0;
  PostParams hparams{0.25f, 0.45f, MAX_OUT, 0};
  // pinned mirror of `results` (filled inside the graph)
  void* h_results = nullptr;
  f16* h_probs = nullptr;             // classify: pinned [B][nc] probabilities (in the graph)
  float* h_out = nullptr;
  int* h_cnt = nullptr;
  int* h_rawcnt = nullptr;
  int cstride = 6;
  int lastDecode = -1;
  DecodeArgs dec{};
  // graphs
  std::vector<hipGraphExec_t> graphs;
  std::vector<float> execMs;
  hipGraphExec_t frameGraph = nullptr;
  // The same frame graph with the one-block NMS: yolo_frame_run / _launch take it while the
  // previous frame had at most NMS_BLOCK_MAX candidates in every slot (the one launch beats
  // the multi-block pipeline's six on sparse frames; results are identical either way).
  hipGraphExec_t frameGraphBlock = nullptr;
  std::vector<uint8_t*> stageDev;     // yolo_stage_frames / _jpeg: per-slot device raw frames
  std::vector<size_t> stageCap;
  // yolo_stage_jpeg: two pinned staging areas (coefficients + descriptors) used in turn, each
  // rewritten only after its last copy has run; the device mirror and the IDCT sample planes
  struct JpegStage {
    uint8_t* host = nullptr;
    size_t cap = 0;
    hipEvent_t copied = nullptr;
    bool pending = false;
  };
  JpegStage jpegStage[2];
  int jpegNext = 0;
  uint8_t* jpegDev = nullptr;
  size_t jpegDevCap = 0;
  uint8_t* jpegSamples = nullptr;
  size_t jpegSamplesCap = 0;
  std::vector<int> jpegH, jpegW;       // per slot: the frame yolo_decode_jpeg left in its
                                       // staging buffer (0: none / failed / overwritten)
  // The JPEG decode's copies and kernels run on a stream of their own, beside the network of
  // the batch in flight.  It starts after `readDone` (the last letterbox, on the engine
  // stream, that read the staging frames); the engine stream's next reader of decoded frames
  // waits for `decodeDone`.
  hipStream_t decodeSt = nullptr;
  hipEvent_t readDone = nullptr, decodeDone = nullptr;
  bool decodePending = false;
  bool capBlock = false;              // capture(): post() records the one-block NMS
  int frameB = 0;
  // the frame graph's device sources and sizes (for stage timing outside the graph)
  std::vector<std::pair<const uint8_t*, SlotGeom>> frameSrc;
  std::vector<int> frameH, frameW;
  std::vector<SlotGeom> slots;
  std::vector<SlotGeom> frameSlots;
  // branch concurrency: ops are spread over the main stream and NSIDE side streams by a
  // list scheduler over their buffer read/write sets; captured graphs inherit the edges
  static constexpr int NSIDE = 3;
  std::vector<hipStream_t> side;
  std::vector<int> opStream;               // 0 = main, 1..NSIDE = side[i-1]
  std::vector<std::vector<int>> opWaits;   // ops (on other streams) to wait for first
  std::vector<char> opRecord;              // record an event after this op
  std::vector<hipEvent_t> opEvent;
  hipEvent_t forkEv = nullptr;
  std::vector<hipEvent_t> joinEv;

  ~Engine() { release(); }

  View view(int t) const {
    const TenDesc& T = g.tens[t];
    const BufDesc& Bd = g.bufs[T.buf];
    return View{bufp[T.buf], Bd.H, Bd.W, Bd.C, T.coff, T.C};
  }

  void release() {
    if (st) (void)hipStreamSynchronize(st);
    if (decodeSt) (void)hipStreamSynchronize(decodeSt);
    for (auto& ge : graphs)
      if (ge) (void)hipGraphExecDestroy(ge);
    graphs.clear();
    for (uint8_t* p : stageDev)
      if (p) (void)hipFree(p);
    stageDev.clear();
    stageCap.clear();
    for (JpegStage& js : jpegStage) {
      if (js.copied) (void)hipEventSynchronize(js.copied);
      if (js.host) (void)hipHostFree(js.host);
      if (js.copied) (void)hipEventDestroy(js.copied);
      js = JpegStage{};
    }
    if (jpegDev) (void)hipFree(jpegDev);
    if (jpegSamples) (void)hipFree(jpegSamples);
    jpegDev = jpegSamples = nullptr;
    jpegDevCap = jpegSamplesCap = 0;
    if (frameGraph) (void)hipGraphExecDestroy(frameGraph);
    if (frameGraphBlock) (void)hipGraphExecDestroy(frameGraphBlock);
    frameGraph = frameGraphBlock = nullptr;
    void* dptrs[] = {arena, weights, bias, cand, nmsCount, nmsScratch, nmsWork, results, outidx, masks,
                     params, splitWs, splitCnt};
    for (void* p : dptrs)
      if (p) (void)hipFree(p);
    arena = nullptr; weights = nullptr; bias = nullptr; cand = nullptr; nmsCount = nullptr;
    nmsScratch = nullptr; nmsWork = nullptr; results = nullptr; outdets = nullptr; outidx = nullptr; outcnt = nullptr;
    rawcnt = nullptr;
    masks = nullptr; params = nullptr; splitWs = nullptr; splitCnt = nullptr;
    splitWsBytes = splitCntN = 0;
    if (h_results) (void)hipHostFree(h_results);
    if (h_probs) (void)hipHostFree(h_probs);
    h_probs = nullptr;
    h_results = nullptr; h_out = nullptr; h_cnt = nullptr; h_rawcnt = nullptr;
    for (hipEvent_t e : opEvent)
      if (e) (void)hipEventDestroy(e);
    opEvent.clear();
    for (hipEvent_t e : joinEv)
      if (e) (void)hipEventDestroy(e);
    joinEv.clear();
    if (forkEv) (void)hipEventDestroy(forkEv);
    forkEv = nullptr;
    for (hipStream_t s : side)
      if (s) (void)hipStreamDestroy(s);
    side.clear();
    if (st) (void)hipStreamDestroy(st);
    st = nullptr;
    if (decodeSt) (void)hipStreamDestroy(decodeSt);
    if (readDone) (void)hipEventDestroy(readDone);
    if (decodeDone) (void)hipEventDestroy(decodeDone);
    decodeSt = nullptr;
    readDone = decodeDone = nullptr;
    decodePending = false;
  }

  // Both streams idle (before a buffer either may use is freed).
  void syncAll() {
    HCK(hipStreamSynchronize(st));
    if (decodeSt) HCK(hipStreamSynchronize(decodeSt));
  }

  void ensureDecodeStream() {
    if (decodeSt) return;
    HCK(hipStreamCreateWithFlags(&decodeSt, hipStreamNonBlocking));
    HCK(hipEventCreateWithFlags(&readDone, hipEventDisableTiming));
    HCK(hipEventCreateWithFlags(&decodeDone, hipEventDisableTiming));
    HCK(hipEventRecord(readDone, st));   // everything already queued may read staging frames
  }

  // The engine stream's next reader or writer of staging frames orders after the decodes.
  void waitDecoded() {
    if (decodePending) HCK(hipStreamWaitEvent(st, decodeDone, 0));
  }

  // ---------------------------------------------------------------- stream plan
  // Each op's accesses are (buffer, channel range, write?) sets; op j depends on an
  // earlier op i when they touch overlapping channel ranges of one buffer and either
  // writes.  A list scheduler then keeps dependency chains on one stream and starts an
  // independent op on the stream that went idle earliest, waiting only for the latest
  // dependency on each other stream.  Decode (one launch for all levels) depends on every
  // head tensor, and post-processing joins all streams.
  // Buffer-region access sets of every op (what it reads and writes), the basis of both
  // the eager multi-stream plan and the graph DAG.  A fused pool chain's head carries the
  // accesses of its followers.
  struct Acc { int buf, c0, c1; bool w; };
  std::vector<std::vector<Acc>> acc;
  void computeAccesses() {
    const int n = (int)ops.size();
    acc.assign(n, {});
    auto add = [&](int k, int t, bool w) {
      if (t < 0) return;
      const TenDesc& T = g.tens[t];
      acc[k].push_back({T.buf, T.coff, T.coff + T.C, w});
    };
    for (int k = 0; k < n; k++) {
      const OpDesc& op = ops[k];
      const int at = op.chain < 0 ? k - 1 - (k >= 2 && ops[k - 1].chain < 0 ? 1 : 0) : k;
      switch (op.kind) {
        case CONV: add(at, op.a, false); add(at, op.b, false); add(at, op.out, true); break;
        case ADD: add(at, op.a, false); add(at, op.b, false); add(at, op.out, true); break;
        case DECODE:
        case DECODESEG:
        case DECODEOBB:
          if (k == lastDecode)
            for (const OpDesc& d : ops)
              if (isDecode(d.kind)) { add(k, d.a, false); add(k, d.b, false); add(k, d.out, false); }
          break;
        case MASKS: break;
        default: add(at, op.a, false); add(at, op.out, true); break;
      }
    }
  }
  bool conflict(int i, int j) const {
    for (const Acc& x : acc[i])
      for (const Acc& y : acc[j])
        if (x.buf == y.buf && x.c0 < y.c1 && y.c0 < x.c1 && (x.w || y.w)) return true;
    return false;
  }

  // Graph DAG: deps[j] = earlier ops whose accesses conflict with op j's, transitively
  // reduced (an edge implied by a path through another dependency is dropped).
  std::vector<std::vector<int>> dagDeps;
  void planDag() {
    computeAccesses();
    const int n = (int)ops.size();
    const int words = (n + 63) / 64;
    std::vector<std::vector<uint64_t>> anc(n, std::vector<uint64_t>(words, 0));
    dagDeps.assign(n, {});
    for (int j = 0; j < n; j++) {
      if (acc[j].empty()) continue;
      std::vector<int> d;
      for (int i = j - 1; i >= 0; i--)
        if (!acc[i].empty() && conflict(i, j)) d.push_back(i);
      // latest first: a dependency already reachable from a kept one is implied
      std::vector<uint64_t> reach(words, 0);
      for (int i : d) {
        if ((reach[i >> 6] >> (i & 63)) & 1) continue;
        dagDeps[j].push_back(i);
        reach[i >> 6] |= 1ull << (i & 63);
        for (int w = 0; w < words; w++) reach[w] |= anc[i][w];
      }
      anc[j] = reach;
    }
  }

  void planStreams() {
    computeAccesses();
    const int n = (int)ops.size();
    const int NS = 1 + NSIDE;
    opStream.assign(n, 0);
    opWaits.assign(n, {});
    opRecord.assign(n, 0);
    std::vector<int> last(NS, -1);
    for (int j = 0; j < n; j++) {
      std::vector<int> latest(NS, -1);   // latest dependency per stream
      int L = -1;
      for (int i = 0; i < j; i++)
        if (conflict(i, j)) {
          latest[opStream[i]] = std::max(latest[opStream[i]], i);
          L = std::max(L, i);
        }
      int s;
      if (L >= 0 && last[opStream[L]] == L) {
        s = opStream[L];                  // continue the chain
      } else {
        s = 0;                            // the stream that went idle earliest
        for (int q = 1; q < NS; q++)
          if (last[q] < last[s]) s = q;
      }
      opStream[j] = s;
      last[s] = j;
      for (int q = 0; q < NS; q++)
        if (q != s && latest[q] >= 0) {
          opWaits[j].push_back(latest[q]);
          opRecord[latest[q]] = 1;
        }
    }
  }

  void createStreams() {
    side.assign(NSIDE, nullptr);
    for (auto& s : side) HCK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    opEvent.assign(ops.size(), nullptr);
    for (size_t k = 0; k < ops.size(); k++)
      if (opRecord[k]) HCK(hipEventCreateWithFlags(&opEvent[k], hipEventDisableTiming));
    HCK(hipEventCreateWithFlags(&forkEv, hipEventDisableTiming));
    joinEv.assign(NSIDE, nullptr);
    for (auto& e : joinEv) HCK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  }

  // ---------------------------------------------------------------- load
  void load(const std::string& dir, int maxB, bool fuse) {
    std::string err;
    if (maxB < 1) throw Failure("max_batch must be >= 1");
    if (!parseGraph(dir, g, err) || !validateGraph(g, err)) throw Failure(err);
    B = maxB;
    ops = g.ops;
    if (fuse) {
      fuseAdds(ops);
      // SPPF: three chained MAXPOOL5 ops -> one launch (the plane must fit the LDS budget)
      for (size_t i = 0; i + 2 < ops.size(); i++) {
        OpDesc &p0 = ops[i], &p1 = ops[i + 1], &p2 = ops[i + 2];
        if (p0.kind != MAXPOOL5 || p1.kind != MAXPOOL5 || p2.kind != MAXPOOL5) continue;
        // exporters register a fresh tensor id per use, so match the views themselves
        auto same = [&](int t0, int t1) {
          const TenDesc &u = g.tens[t0], &v = g.tens[t1];
          return u.buf == v.buf && u.coff == v.coff && u.C == v.C;
        };
        if (!same(p1.a, p0.out) || !same(p2.a, p1.out) || p0.chain || p1.chain || p2.chain) continue;
        const BufDesc& xb = g.bufs[g.tens[p0.a].buf];
        if (sppfPoolLds(xb.H, xb.W) > 64 * 1024) continue;
        p0.chain = 3;
        p1.chain = p2.chain = -1;
      }
    }
    for (size_t i = 0; i < ops.size(); i++) {
      const OpDesc& op = ops[i];
      if (op.kind == CONV && op.g == 1 && op.Cin == 3 && op.b >= 0)
        throw Failure(fmt("op %zu: first conv with a residual is not supported", i));
      if (op.kind == CONV && op.b >= 0) {
        const TenDesc& r = g.tens[op.b];
        const TenDesc& y = g.tens[op.out];
        if (g.bufs[r.buf].H != g.bufs[y.buf].H || g.bufs[r.buf].W != g.bufs[y.buf].W || r.C != y.C ||
            r.coff % 8 || g.bufs[r.buf].C % 8)
          throw Failure(fmt("op %zu: residual view does not match the output", i));
      }
      if (op.kind == CONV && op.g == 1 && op.Cin != 3) {
        const BufDesc& xb = g.bufs[g.tens[op.a].buf];
        if (!convGemmFits((long)B * xb.H * xb.W * xb.C * 2, (long)op.Cout * op.k * op.k * op.Cin * 2))
          throw Failure(fmt("op %zu: conv input or weights reach 2 GiB at batch %d", i, B));
      }
      if (isDecode(op.kind)) lastDecode = (int)i;
    }
    // weights: read, check ranges, repack depthwise [C][k*k] -> [k*k][C]
    std::vector<char> wf, bf;
    if (!readFile(dir + "/weights.f16", wf, err) || !readFile(dir + "/bias.f32", bf, err)) throw Failure(err);
    nweights = wf.size() / 2;
    nbias = bf.size() / 4;
    f16* w = (f16*)wf.data();
    for (size_t i = 0; i < g.ops.size(); i++) {
      const OpDesc& op = g.ops[i];
      if (op.kind != CONV) continue;
      size_t cnt = (size_t)op.Cout * op.k * op.k * (op.Cin / op.g);
      if (op.woff + cnt > nweights || op.boff + (size_t)op.Cout > nbias)
        throw Failure(fmt("op %zu: weight/bias offsets exceed weights.f16 / bias.f32", i));
      if (op.g > 1) {
        int C = op.Cin, KK = op.k * op.k;
        std::vector<f16> t((size_t)C * KK);
        for (int c = 0; c < C; c++)
          for (int r = 0; r < KK; r++) t[(size_t)r * C + c] = w[op.woff + (size_t)c * KK + r];
        memcpy(w + op.woff, t.data(), t.size() * sizeof(f16));
      }
    }
    HCK(hipStreamCreate(&st));
    attentionInit();
    HCK(hipMalloc(&weights, std::max<size_t>(wf.size(), 16)));
    HCK(hipMalloc(&bias, std::max<size_t>(bf.size(), 16)));
    HCK(hipMemcpy(weights, wf.data(), wf.size(), hipMemcpyHostToDevice));
    HCK(hipMemcpy(bias, bf.data(), bf.size(), hipMemcpyHostToDevice));
    // activation arena
    size_t total = 0;
    std::vector<size_t> offs;
    for (const BufDesc& b : g.bufs) {
      offs.push_back(total);
      total += ((size_t)B * b.H * b.W * b.C * sizeof(f16) + 255) & ~(size_t)255;
    }
    HCK(hipMalloc(&arena, total));
    HCK(hipMemset(arena, 0, total));
    for (size_t i = 0; i < g.bufs.size(); i++) bufp.push_back((f16*)((char*)arena + offs[i]));
    // post-processing state
    const int A = std::max(g.numAnchors, 1);   // graphs without DECODE keep 1-slot buffers
    cstride = g.detStride;
    HCK(hipMalloc(&cand, (size_t)B * A * cstride * sizeof(float)));
    HCK(hipMalloc(&nmsCount, (size_t)B * sizeof(int)));
    HCK(hipMemset(nmsCount, 0, (size_t)B * sizeof(int)));
    HCK(hipMalloc(&nmsScratch, (size_t)B * nmsScratchBytes(A)));
    if (g.numAnchors > 0 && !nmsBlock) {
      HCK(hipMalloc(&nmsWork, (size_t)B * sizeof(NmsImage)));
      HCK(hipMemset(nmsWork, 0, (size_t)B * sizeof(NmsImage)));
    }
    detOff = ((size_t)2 * B * sizeof(int) + 255) & ~(size_t)255;
    const size_t resBytes = detOff + (size_t)B * MAX_OUT * g.outK * sizeof(float);
    HCK(hipMalloc(&results, resBytes));
    HCK(hipMemset(results, 0, resBytes));
    outcnt = (int*)results;
    rawcnt = outcnt + B;
    outdets = (float*)((char*)results + detOff);
    HCK(hipMalloc(&outidx, (size_t)B * MAX_OUT * sizeof(int)));
    HCK(hipMemset(cand, 0, (size_t)B * A * cstride * sizeof(float)));
    HCK(hipMemset(outidx, 0, (size_t)B * MAX_OUT * sizeof(int)));
    if (g.protoTen >= 0) {
      const BufDesc& pb = g.bufs[g.tens[g.protoTen].buf];
      HCK(hipMalloc(&masks, (size_t)B * MAX_OUT * pb.H * pb.W));
      HCK(hipMemset(masks, 0, (size_t)B * MAX_OUT * pb.H * pb.W));
    }
    HCK(hipMalloc(&params, sizeof(PostParams)));
    HCK(hipMemcpy(params, &hparams, sizeof(PostParams), hipMemcpyHostToDevice));
    HCK(hipHostMalloc(&h_results, resBytes, hipHostMallocDefault));
    memset(h_results, 0, resBytes);
    h_cnt = (int*)h_results;
    h_rawcnt = h_cnt + B;
    h_out = (float*)((char*)h_results + detOff);
    if (g.cls) {
      HCK(hipHostMalloc((void**)&h_probs, (size_t)B * g.nc * sizeof(f16), hipHostMallocDefault));
      memset(h_probs, 0, (size_t)B * g.nc * sizeof(f16));
    }
    // decode levels in op order
    dec = DecodeArgs{};
    int base = 0;
    for (const OpDesc& op : ops) {
      if (!isDecode(op.kind)) continue;
      DecodeLevel& L = dec.lv[dec.nlev++];
      L.box = view(op.a);
      L.cls = view(op.b);
      L.coef = op.kind != DECODE ? view(op.out) : View{nullptr, 0, 0, 0, 0, 0};
      L.H = L.box.H;
      L.W = L.box.W;
      L.stride = op.stride;
      L.base = base;
      base += L.H * L.W;
    }
    dec.A = A;
    dec.nc = g.nc;
    dec.nm = g.seg ? g.nm : 0;
    dec.obb = g.obb ? 1 : 0;
    slots.assign(B, SlotGeom{});
    HCK(hipDeviceSynchronize());
  }

  // ---------------------------------------------------------------- dispatch
  void runOp(int k, int Bn, hipStream_t s = nullptr) {
    if (!s) s = st;
    const OpDesc& op = ops[k];
    switch (op.kind) {
      case CONV: {
        View x = view(op.a), y = view(op.out);
        View r{};
        const View* rp = nullptr;
        if (op.b >= 0) { r = view(op.b); rp = &r; }
        const f16* w = weights + op.woff;
        const float* b = bias + op.boff;
        if (op.g == 1 && op.Cin == 3)
          launchConvFirst(x, y, w, b, op.s, op.p, op.act, Bn, s);
        else if (op.g == 1 && specialConvCfg(op.cfg) && specialConvOk(op.cfg, x, y, rp, op.k, op.s, op.p))
          launchSpecialConv(op.cfg, x, y, rp, w, b, op.act, Bn, s);   // (else: the GEMM's default tile)
        else if (op.g == 1)
          launchConvGemm(op.cfg, x, y, rp, w, b, op.k, op.s, op.p, op.act, Bn, op.split,
                         op.wsOff >= 0 ? splitWs + op.wsOff : nullptr,
                         op.cntOff >= 0 ? splitCnt + op.cntOff : nullptr, s, op.tail);
        else
          launchDwConv(x, y, rp, w, b, op.k, op.s, op.p, op.act, Bn, s);
        break;
      }
      case ADD: launchAdd(view(op.a), view(op.b), view(op.out), Bn, s); break;
      case MAXPOOL5:
        if (op.chain == 3)
          launchSppfPool(view(op.a), view(op.out), view(ops[k + 1].out), view(ops[k + 2].out), Bn, s);
        else
          launchMaxPool5(view(op.a), view(op.out), Bn, s);
        break;
      case UPSAMPLE2: launchUpsample2(view(op.a), view(op.out), Bn, s); break;
      case COPYC: launchCopyC(view(op.a), view(op.out), Bn, s); break;
      case PS2: launchPS2(view(op.a), view(op.out), Bn, s); break;
      case ATTN: launchAttention(view(op.a), view(op.out), op.heads, op.kd, op.hd, Bn, s); break;
      case DECODE:
      case DECODESEG:
      case DECODEOBB:
        // all levels decode in one launch, issued at the last DECODE op (every head
        // tensor is final by then)
        if (k == lastDecode) launchDecode(dec, cand, nmsScratch, nmsCount, params, Bn, s);
        break;
      case GAP: launchGap(view(op.a), view(op.out), Bn, s); break;
      case SOFTMAX: launchSoftmaxCh(view(op.a), view(op.out), Bn, s); break;
      default: break;   // MASKS is declarative; assembly runs after NMS
    }
  }

  // ---------------------------------------------------------------- launch units
  // forward() runs the ops as a list of units: one op, or a group of independent ops of one
  // kernel kind launched together (GEMM convs sharing a tile config and K mode, depthwise
  // convs, channel copies).  A group's launch computes every member exactly as a launch of
  // it alone does (grouped kernels only partition their blocks), so grouping changes launch
  // counts, never results.
  enum { GK_NONE = 0, GK_GEMM, GK_DW, GK_COPY, GK_ATTN };   // GK_ATTN: an attention + the copies it carries
  struct Unit {
    std::vector<int> ops;
    int kind = GK_NONE;
  };
  std::vector<Unit> units;
  int groupKind(int k) const {
    const OpDesc& op = ops[k];
    if (op.chain < 0) return GK_NONE;
    if (op.kind == COPYC) return GK_COPY;
    if (op.kind != CONV) return GK_NONE;
    if (op.g > 1) return GK_DW;
    if (op.Cin == 3 || op.tail >= 0) return GK_NONE;
    return GK_GEMM;   // a conv tuned to a special kernel too: a group must then beat that kernel
  }
  ConvJob convJob(int k) {
    const OpDesc& op = ops[k];
    jobRes.push_back(op.b >= 0 ? view(op.b) : View{});
    return ConvJob{view(op.a), view(op.out), op.b >= 0 ? &jobRes.back() : nullptr, weights + op.woff,
                   bias + op.boff, op.k, op.s, op.p, op.act};
  }
  std::deque<View> jobRes;   // residual views the jobs of one launch point at
  void launchGroup(int kind, const std::vector<int>& m, int cfg, int Bn, hipStream_t s) {
    jobRes.clear();
    if (kind == GK_COPY) {
      View xs[COPY_GROUP], ys[COPY_GROUP];
      for (size_t i = 0; i < m.size(); i++) { xs[i] = view(ops[m[i]].a); ys[i] = view(ops[m[i]].out); }
      launchCopyCGroup(xs, ys, (int)m.size(), Bn, s);
      return;
    }
    ConvJob jobs[GEMM_GROUP > DW_GROUP ? GEMM_GROUP : DW_GROUP];
    for (size_t i = 0; i < m.size(); i++) jobs[i] = convJob(m[i]);
    if (kind == GK_DW)
      launchDwConvGroup(jobs, (int)m.size(), Bn, s);
    else
      launchConvGemmGroup(cfg, jobs, (int)m.size(), Bn, s);
  }
  void runUnit(const Unit& u, int Bn, hipStream_t s = nullptr) {
    if (!s) s = st;
    if (u.kind == GK_ATTN) {
      const OpDesc& a = ops[u.ops[0]];
      View xs[COPY_GROUP], ys[COPY_GROUP];
      for (size_t i = 1; i < u.ops.size(); i++) {
        xs[i - 1] = view(ops[u.ops[i]].a);
        ys[i - 1] = view(ops[u.ops[i]].out);
      }
      launchAttention(view(a.a), view(a.out), a.heads, a.kd, a.hd, Bn, s, xs, ys, (int)u.ops.size() - 1);
      return;
    }
    bool together = u.ops.size() > 1;
    if (together && u.kind == GK_GEMM)   // (per-op overrides since planning launch one by one)
      for (int i : u.ops)
        together = together && ops[i].cfg == ops[u.ops[0]].cfg && ops[i].split == 1 && ops[i].tail < 0;
    if (!together) {
      for (int i : u.ops)
        if (ops[i].chain >= 0) runOp(i, Bn, s);
      return;
    }
    launchGroup(u.kind, u.ops, ops[u.ops[0]].cfg, Bn, s);
  }
  static int groupMax(int kind) { return kind == GK_GEMM ? GEMM_GROUP : kind == GK_DW ? DW_GROUP : COPY_GROUP; }

  // Groups ops that no dependency orders, in two passes over the unit list (each unit is
  // atomic: its accesses are its members' accesses, its place its first member's place).
  // A single-op unit takes later single-op units of its kind (within 40 units) that conflict
  // with neither the group nor any unit they would move ahead of.  Pass 1 only takes ops of
  // the same shape class (GEMM: same kernel size, stride and output width -- the levels of a
  // detection head, the twin 1x1 convs of a C3k block); pass 2 any GEMM conv of the same K
  // mode.  Depthwise convs and copies always group; a GEMM group must find one tile config
  // that runs it faster than its members' own tuned configs (GEMM tiles or special kernels)
  // launched one after another (timed at the max batch like the autotuner; the full
  // candidate set first, then shorter prefixes).  Without tuning GEMM ops stay single.
  bool unitConflict(const Unit& a, const Unit& b) const {
    for (int i : a.ops)
      for (int j : b.ops)
        if (conflict(i, j)) return true;
    return false;
  }
  bool sameClass(int i, int j) const {
    const OpDesc &a = ops[i], &b = ops[j];
    return a.k == b.k && a.s == b.s && a.Cout == b.Cout && a.act == b.act;
  }
  void mergePass(bool strict, bool tune, hipEvent_t e0, hipEvent_t e1) {
    auto timeIt = [&](auto&& launch) {
      for (int r = 0; r < 2; r++) launch();
      float t[7];
      for (int r = 0; r < 7; r++) {
        HCK(hipEventRecord(e0, st));
        launch();
        HCK(hipEventRecord(e1, st));
        HCK(hipEventSynchronize(e1));
        HCK(hipEventElapsedTime(&t[r], e0, e1));
      }
      std::sort(t, t + 7);
      return t[3];
    };
    std::vector<Unit> out;
    std::vector<char> taken(units.size(), 0);
    for (size_t a = 0; a < units.size(); a++) {
      if (taken[a]) continue;
      taken[a] = 1;
      Unit u = units[a];
      const int kind = u.ops.size() == 1 ? groupKind(u.ops[0]) : GK_NONE;
      if (kind == GK_NONE || (kind == GK_GEMM && !tune) || (kind != GK_GEMM && !strict)) {
        out.push_back(u);
        continue;
      }
      const int k = u.ops[0];
      std::vector<size_t> cand;
      for (size_t b = a + 1; b < units.size() && b <= a + 40 && (int)cand.size() + 1 < groupMax(kind); b++) {
        if (taken[b] || units[b].ops.size() != 1) continue;
        const int j = units[b].ops[0];
        if (groupKind(j) != kind || (strict && kind == GK_GEMM && !sameClass(k, j))) continue;
        bool ok = !unitConflict(u, units[b]);
        for (size_t c : cand) ok = ok && !unitConflict(units[c], units[b]);
        for (size_t c = a + 1; c < b && ok; c++)
          if (!taken[c] && std::find(cand.begin(), cand.end(), c) == cand.end() && unitConflict(units[c], units[b]))
            ok = false;
        if (ok) cand.push_back(b);
      }
      if (kind == GK_GEMM) {
        // the longest prefix of the candidates that one tile config runs faster together
        size_t keep = 0;
        int keepCfg = -1;
        for (size_t m = cand.size(); m >= 1 && keepCfg < 0; m--) {
          std::vector<int> grp{k};
          for (size_t i = 0; i < m; i++) grp.push_back(units[cand[i]].ops[0]);
          const float sep = timeIt([&] { for (int i : grp) runOp(i, B); });
          jobRes.clear();
          std::vector<ConvJob> jobs;
          for (int i : grp) jobs.push_back(convJob(i));
          float best = sep;
          for (int cfg = 0; cfg < numTileConfigs(); cfg++) {
            bool fits = convGroupOk(cfg, jobs.data(), (int)jobs.size());
            for (int i : grp) {
              const View y = view(ops[i].out);
              fits = fits && tileOk(cfg, B * y.H * y.W, ops[i].Cout, ops[i].k * ops[i].k * ops[i].Cin);
            }
            if (!fits) continue;
            const float t = timeIt([&] { launchConvGemmGroup(cfg, jobs.data(), (int)jobs.size(), B, st); });
            if (t < best) { best = t; keepCfg = cfg; keep = m; }
          }
        }
        cand.resize(keep);
        if (keepCfg >= 0) {
          ops[k].cfg = keepCfg;
          ops[k].split = 1;
          for (size_t c : cand) {
            OpDesc& o = ops[units[c].ops[0]];
            o.cfg = keepCfg;
            o.split = 1;
          }
        }
      }
      for (size_t c : cand) {
        taken[c] = 1;
        u.ops.push_back(units[c].ops[0]);
      }
      if (u.ops.size() > 1) u.kind = kind;
      out.push_back(u);
    }
    units = out;
  }
  // A unit of channel copies (one COPYC, or a copy group) moves into the launch of a later
  // attention op (within the next 8 units) that none of the copies conflicts with, when no
  // unit in between conflicts with them either: the copies then run as the attention
  // launch's trailing blocks.  C2PSA gathers each head's V slice of the qkv tensor this way
  // for its positional conv, independent of the attention that reads the same tensor.
  void carryCopies() {
    std::vector<Unit> out;
    for (size_t a = 0; a < units.size(); a++) {
      const Unit& u = units[a];
      bool copies = !u.ops.empty() && u.ops.size() <= (size_t)COPY_GROUP;
      for (int i : u.ops) copies = copies && groupKind(i) == GK_COPY;
      if (copies) {
        for (size_t b = a + 1; b < units.size() && b <= a + 8; b++) {
          const Unit& v = units[b];
          if (v.ops.size() == 1 && ops[v.ops[0]].kind == ATTN && ops[v.ops[0]].chain >= 0 && !unitConflict(u, v)) {
            Unit m{{v.ops[0]}, GK_ATTN};
            m.ops.insert(m.ops.end(), u.ops.begin(), u.ops.end());
            units[b] = m;      // the copies' place becomes the attention's
            copies = false;
            break;
          }
          if (unitConflict(u, v)) break;
        }
        if (!copies) continue;   // carried
      }
      out.push_back(u);
    }
    units = out;
  }
  void planUnits(bool tune) {
    computeAccesses();
    units.clear();
    for (int k = 0; k < (int)ops.size(); k++) units.push_back({{k}, GK_NONE});
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (tune) {
      HCK(hipEventCreate(&e0));
      HCK(hipEventCreate(&e1));
    }
    mergePass(true, tune, e0, e1);
    mergePass(false, tune, e0, e1);
    carryCopies();
    for (Unit& u : units)
      for (int i : u.ops) ops[i].wsOff = ops[i].cntOff = -1;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    HCK(hipGetLastError());
    if (getenv("YOLO_PRINT_UNITS")) {   // the plan, for inspection: grouped units only
      int launches = 0;
      for (const Unit& u : units) launches += u.ops.size() > 1 || ops[u.ops[0]].chain >= 0;
      fprintf(stderr, "yolo: %zu ops in %d launches (B=%d)\n", ops.size(), launches, B);
      const bool all = atoi(getenv("YOLO_PRINT_UNITS")) > 1;
      for (const Unit& u : units)
        if (u.ops.size() > 1 || (all && ops[u.ops[0]].chain >= 0)) {
          fprintf(stderr, "  group kind %d cfg %d:", u.kind, ops[u.ops[0]].cfg);
          for (int i : u.ops) fprintf(stderr, " %d", i);
          fprintf(stderr, "\n");
        }
    }
  }

  void post(int Bn) {
    if (g.cls) {   // no decode/NMS: the probabilities go to pinned memory (engine/engine.cu:1458)
      HCK(hipMemcpyAsync(h_probs, bufp[g.tens[g.probsTen].buf], (size_t)Bn * g.nc * sizeof(f16),
                         hipMemcpyDeviceToHost, st));
      return;
    }
    if (g.numAnchors == 0) return;   // no detection head (single-op graphs)
    const bool multi = nmsWork && !capBlock;
    if (g.obb && multi)
      launchNmsObbMulti(cand, nmsScratch, nmsCount, g.numAnchors, outdets, outidx, outcnt, rawcnt, params, nmsWork,
                        Bn, st);
    else if (g.obb)
      launchNmsObb(cand, nmsScratch, nmsCount, g.numAnchors, outdets, outidx, outcnt, rawcnt, params, Bn, st);
    else if (multi)
      launchNmsMulti(cand, nmsScratch, nmsCount, g.numAnchors, cstride, outdets, outidx, outcnt, rawcnt, params,
                     nmsWork, Bn, st);
    else
      launchNms(cand, nmsScratch, nmsCount, g.numAnchors, cstride, outdets, outidx, outcnt, rawcnt, params, Bn, st);
    if (g.protoTen >= 0) {
      View pr = view(g.protoTen);
      launchMasks(pr, cand, cstride, g.numAnchors, g.nm, outidx, outcnt, outdets, masks,
                  (float)pr.W / g.bufs[g.tens[0].buf].W, (float)pr.H / g.bufs[g.tens[0].buf].H, Bn, st);
    }
    HCK(hipMemcpyAsync(h_results, results, detOff + (size_t)Bn * MAX_OUT * g.outK * sizeof(float),
                       hipMemcpyDeviceToHost, st));
  }

  // `branches`: use the side-stream plan (eager execution only).  Graphs never capture the
  // fork/join plan (capturing it crashed inside hipStreamEndCapture on this ROCm 7.2 image;
  // the cause was not isolated): they get branch concurrency from the explicit DAG of
  // per-op child graphs built in capture() instead.
  void forward(int Bn, bool branches = true) {
    if (side.empty() || !branches) {
      for (const Unit& u : units) runUnit(u, Bn);
    } else {
      auto strm = [&](int s) { return s == 0 ? st : side[s - 1]; };
      HCK(hipEventRecord(forkEv, st));
      for (hipStream_t s : side) HCK(hipStreamWaitEvent(s, forkEv, 0));
      for (size_t k = 0; k < ops.size(); k++) {
        hipStream_t s = strm(opStream[k]);
        for (int w : opWaits[k]) HCK(hipStreamWaitEvent(s, opEvent[w], 0));
        if (ops[k].chain >= 0) runOp((int)k, Bn, s);
        if (opRecord[k]) HCK(hipEventRecord(opEvent[k], s));
      }
      for (int q = 0; q < NSIDE; q++) {
        HCK(hipEventRecord(joinEv[q], side[q]));
        HCK(hipStreamWaitEvent(st, joinEv[q], 0));
      }
    }
    post(Bn);
  }

  // ---------------------------------------------------------------- split-K scratch
  // Grow the shared split-K buffers to at least `bytes` / `ncnt` (counters zeroed).  Only
  // called before any graph is captured: graphs hold raw pointers into these buffers.
  void ensureSplitScratch(size_t bytes, size_t ncnt) {
    if (bytes > splitWsBytes) {
      if (splitWs) HCK(hipFree(splitWs));
      splitWs = nullptr;
      HCK(hipMalloc(&splitWs, bytes));
      splitWsBytes = bytes;
    }
    if (ncnt > splitCntN) {
      if (splitCnt) HCK(hipFree(splitCnt));
      splitCnt = nullptr;
      HCK(hipMalloc(&splitCnt, ncnt * sizeof(int)));
      HCK(hipMemset(splitCnt, 0, ncnt * sizeof(int)));
      splitCntN = ncnt;
    }
  }
  // Give every split op its own workspace and counter range (sized at the max batch), so
  // ops on concurrent streams never share partials.
  void assignSplits() {
    size_t wsTot = 0, cntTot = 0;
    for (OpDesc& op : ops) {
      op.wsOff = op.cntOff = -1;
      if (op.kind != CONV || op.g != 1 || op.Cin == 3 || op.split == 1 || op.split == -1 || specialConvCfg(op.cfg))
        continue;
      View y = view(op.out);
      const int M = B * y.H * y.W, cfg = op.cfg >= 0 ? op.cfg : heuristicTile(M, op.Cout, op.k * op.k * op.Cin);
      const int km = convKMode(cfg, op.k, op.s, op.p, op.Cin);
      op.cfg = cfg;
      op.wsOff = (long)(wsTot / sizeof(float));
      op.cntOff = (long)cntTot;
      wsTot += (splitWorkspaceBytes(cfg, km, M, op.Cout, op.split) + 255) & ~(size_t)255;
      cntTot += splitTiles(cfg, km, M, op.Cout, op.split);
    }
    ensureSplitScratch(wsTot, cntTot);
  }

  // ---------------------------------------------------------------- autotune
  // Time every eligible (tile shape, split-K factor) of every GEMM conv at the max batch
  // (2 warm-up launches, then the median of 7 individually timed ones) and keep the
  // fastest; identical shapes share one measurement.  Splits of every tile are tried only
  // while the tile grid is less than one chip wave.  Tail splits are not candidates: which
  // tiles they split depends on the batch, so an image's sums would depend on the batch it
  // runs in (every choice made here keeps a batch-1 run of a frame bit-identical to its
  // slot in a larger batch); yolo_set_op_split still selects them.  Tail retiles (a smaller
  // tile of the same BK for the rows past the last whole chip wave) are tried on the three
  // fastest plain tiles; they do not change any result bit.
  void autotune() {
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    std::map<std::tuple<int, int, int, int, int, int, int, int>, std::tuple<int, int, int>> cache;
    static const int kSplits[] = {1, 2, 3, 4, 6, 8, 12, 16};
    // YOLO_TUNE_TILES="a,b,..." restricts the candidate tile configs (for A/B studies); the
    // special kernels (halo 1000, resident 1x1 1001, halo-staged 3x3 variants 1100+) take part
    // unless YOLO_TUNE_TILES is set without their entries
    std::vector<char> allowed(numTileConfigs(), 1);
    std::vector<int> specials = {CFG_HALO, CFG_1X1, CFG_1X1S};
    for (int v = 0; v < numTapTiles(); v++) specials.push_back(CFG_TAP + v);
    for (int v = 0; v < numTapWsTiles(); v++) specials.push_back(CFG_TAPWS + v);
    if (const char* lim = getenv("YOLO_TUNE_TILES")) {
      std::fill(allowed.begin(), allowed.end(), 0);
      std::vector<int> keep;
      for (const char* q = lim; *q;) {
        char* end = nullptr;
        const long v = strtol(q, &end, 10);
        if (end == q) break;
        if (v >= 0 && v < numTileConfigs()) allowed[v] = 1;
        if (specialConvCfg((int)v)) keep.push_back((int)v);
        q = *end ? end + 1 : end;
      }
      specials = keep;
    }
    for (size_t k = 0; k < ops.size(); k++) {
      OpDesc& op = ops[k];
      if (op.kind != CONV || op.g != 1 || op.Cin == 3) continue;
      View y = view(op.out);
      const int M = B * y.H * y.W, N = op.Cout, K = op.k * op.k * op.Cin;
      auto key = std::make_tuple(y.H, y.W, op.Cin, op.Cout, op.k, op.s, op.b >= 0 ? 1 : 0, op.act);
      auto it = cache.find(key);
      if (it != cache.end()) {
        std::tie(op.cfg, op.split, op.tail) = it->second;
        continue;
      }
      int best = heuristicTile(M, N, K), bestSplit = 1, bestTail = -1;
      float bestMs = 1e30f;
      auto timeOp = [&] {   // median of 7 timed launches after 2 warm-up ones
        for (int r = 0; r < 2; r++) runOp((int)k, B);
        float t[7];
        for (int r = 0; r < 7; r++) {
          HCK(hipEventRecord(e0, st));
          runOp((int)k, B);
          HCK(hipEventRecord(e1, st));
          HCK(hipEventSynchronize(e1));
          HCK(hipEventElapsedTime(&t[r], e0, e1));
        }
        std::sort(t, t + 7);
        return t[3];   // median: robust to clock ramps and one-off stalls
      };
      std::vector<std::pair<float, int>> plain;   // (ms, cfg) of the unsplit tiles
      for (int cfg = 0; cfg < numTileConfigs(); cfg++) {
        if (!allowed[cfg] || !tileOk(cfg, M, N, K)) continue;
        const int km = convKMode(cfg, op.k, op.s, op.p, op.Cin);
        const int tiles = numTiles(cfg, M, N), P = tileSlots(cfg, km);
        std::vector<int> cands;
        for (int S : kSplits)
          if (S == 1 || (tiles * S <= 1024 && tiles < P)) cands.push_back(S);
        std::sort(cands.begin(), cands.end());
        cands.erase(std::unique(cands.begin(), cands.end()), cands.end());
        for (int S : cands) {
          if (S != 1 && !splitOk(cfg, K, S)) continue;
          op.cfg = cfg;
          op.split = S;
          op.tail = -1;
          op.wsOff = op.cntOff = S != 1 ? 0 : -1;
          if (S != 1) ensureSplitScratch(splitWorkspaceBytes(cfg, km, M, N, S), (size_t)splitTiles(cfg, km, M, N, S));
          const float ms = timeOp();
          if (S == 1) plain.emplace_back(ms, cfg);
          if (ms < bestMs) { bestMs = ms; best = cfg; bestSplit = S; bestTail = -1; }
        }
      }
      std::sort(plain.begin(), plain.end());
      for (size_t i = 0; i < plain.size() && i < 3; i++) {
        const int cfg = plain[i].second;
        for (int tail = 0; tail < numTileConfigs(); tail++) {
          if (!allowed[tail] || !tailOk(cfg, tail, op.k, op.s, op.p, op.Cin, M, N)) continue;
          op.cfg = cfg;
          op.split = 1;
          op.tail = tail;
          op.wsOff = op.cntOff = -1;
          const float ms = timeOp();
          if (ms < bestMs) { bestMs = ms; best = cfg; bestSplit = 1; bestTail = tail; }
        }
      }
      op.tail = -1;
      // the special kernels, where they apply
      View hr{};
      if (op.b >= 0) hr = view(op.b);
      const View* hrp = op.b >= 0 ? &hr : nullptr;
      for (int special : specials) {
        if (!specialConvOk(special, view(op.a), y, hrp, op.k, op.s, op.p)) continue;
        op.cfg = special;
        op.split = 1;
        op.wsOff = op.cntOff = -1;
        const bool handoff = special >= CFG_TAPWS;   // waves that wait on each other: check the waits
        const int failsBefore = handoff ? convSpinFailures() : 0;
        const float ms = timeOp();
        if (handoff && convSpinFailures() != failsBefore) {
          fprintf(stderr, "yolo: op %zu: config %d had an expired wait; not used\n", k, special);
          continue;
        }
        if (ms < bestMs) { bestMs = ms; best = special; bestSplit = 1; bestTail = -1; }
      }
      op.cfg = best;
      op.split = bestSplit;
      op.tail = bestTail;
      op.wsOff = op.cntOff = -1;
      cache[key] = std::make_tuple(best, bestSplit, bestTail);
    }
    HCK(hipGetLastError());
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }

  // ---------------------------------------------------------------- graphs
  // Single-stream capture of whatever `f` enqueues on the engine stream.
  template <class F>
  hipGraph_t captureOne(F&& f) {
    hipGraph_t gr = nullptr;
    HCK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    try {
      f();
    } catch (...) {
      hipGraph_t dummy = nullptr;
      if (hipStreamEndCapture(st, &dummy) == hipSuccess && dummy) (void)hipGraphDestroy(dummy);
      (void)hipGetLastError();
      throw;
    }
    HCK(hipStreamEndCapture(st, &gr));
    return gr;
  }

  void checkFrameInput() const {
    const BufDesc& ib = g.bufs[g.tens[0].buf];
    if (ib.C != 3) throw Failure("letterbox needs a 3-channel input tensor");
    if (g.cls && ib.H != ib.W) throw Failure("classify preprocess needs a square input");
  }

  // A raw frame on the device, in pixel layout fmt, for input slot `slot`.
  struct Staged {
    int slot;
    const uint8_t* src;
    int h, w;
    SlotGeom g;
  };

  // Letterbox (classify: resize + centre crop) of device frames into their input slots: one
  // batched launch for detect-type graphs.
  void preprocessStaged(const std::vector<Staged>& v, int fmt) {
    const BufDesc& ib = g.bufs[g.tens[0].buf];
    if (g.cls) {
      for (const Staged& f : v) {
        const ClsGeom cg = clsGeom(ib.H, f.h, f.w);
        launchPreprocessCls(f.src, f.h, f.w, bufp[g.tens[0].buf] + (size_t)f.slot * ib.H * ib.W * 3, ib.H, cg.rh,
                            cg.rw, cg.top, cg.left, fmt, st);
      }
      if (readDone) HCK(hipEventRecord(readDone, st));
      return;
    }
    std::vector<LetterboxSlot> slots;
    slots.reserve(v.size());
    for (const Staged& f : v)
      slots.push_back(LetterboxSlot{f.src, f.h, f.w, f.g.top, f.g.left, (int)roundf(f.h * f.g.scale),
                                    (int)roundf(f.w * f.g.scale), f.slot, f.g.scale, fmt});
    launchPreprocessBatch(slots.data(), (int)slots.size(), bufp[g.tens[0].buf], ib.H, ib.W, st);
    if (readDone) HCK(hipEventRecord(readDone, st));   // the staging frames are read
  }

  // Frames of slots 0..Bn-1 in pixel layout fmt (PIXEL_BGR / PIXEL_RGBX); host[s], when
  // given, is copied to the device source first.
  void preprocessFrames(int Bn, const std::vector<std::pair<const uint8_t*, SlotGeom>>& frames,
                        const unsigned char* const* host, const int* hs, const int* ws, int fmt = PIXEL_BGR,
                        int firstSlot = 0) {
    std::vector<Staged> v;
    for (int s = 0; s < Bn; s++) {
      if (host && host[s])
        HCK(hipMemcpyAsync((void*)frames[s].first, host[s], (size_t)hs[s] * ws[s] * pixelBytes(fmt),
                           hipMemcpyHostToDevice, st));
      v.push_back(Staged{firstSlot + s, frames[s].first, hs[s], ws[s], frames[s].second});
    }
    preprocessStaged(v, fmt);
  }

  // Device staging buffer of slot s with at least `bytes` (grown after the stream has passed
  // the old one).
  uint8_t* stageBuffer(int s, size_t bytes) {
    if ((int)stageDev.size() < B) {
      stageDev.resize(B, nullptr);
      stageCap.resize(B, 0);
    }
    if (stageCap[s] < bytes) {
      syncAll();
      if (stageDev[s]) HCK(hipFree(stageDev[s]));
      stageDev[s] = nullptr;
      stageCap[s] = 0;
      HCK(hipMalloc(&stageDev[s], bytes));
      stageCap[s] = bytes;
    }
    return stageDev[s];
  }

  int convertDecoded(int Bn, int firstSlot, const std::vector<jpeg::Header>& hd,
                     const std::vector<const int16_t*>& coef, int* status, JpegStage& S, size_t descOff);
  JpegStage& nextStage(size_t bytes);

  void forgetDecoded(int slot) {
    if (slot < (int)jpegH.size()) jpegH[slot] = jpegW[slot] = 0;
  }

  // Grows a device buffer after the stream has passed the old one.
  void growDevice(uint8_t*& p, size_t& cap, size_t bytes) {
    if (cap >= bytes) return;
    const size_t want = std::max(bytes, cap + cap / 2);
    syncAll();
    if (p) HCK(hipFree(p));
    p = nullptr;
    cap = 0;
    HCK(hipMalloc(&p, want));
    cap = want;
  }

  // Batch-Bn graph: [frame prologue] + network + post, by default one single-stream
  // capture.  With a DAG plan (YOLO_DAGGRAPH) every op is captured alone and re-added as
  // kernel nodes whose edges are its buffer conflicts, so the runtime may run independent
  // branches (the head's box/cls chains, neck levels) concurrently.  On ROCm 7.2 the
  // runtime's cross-stream node synchronisation costs more than the overlap gains for
  // these few-microsecond kernels (yolo11n b1: 0.56 ms DAG vs 0.46 ms serial).
  hipGraphExec_t capture(int Bn, const std::vector<std::pair<const uint8_t*, SlotGeom>>* frames,
                         const unsigned char* const* host, const int* hs, const int* ws) {
    hipGraph_t gr = nullptr;
    if (dagDeps.empty()) {
      gr = captureOne([&] {
        if (frames) preprocessFrames(Bn, *frames, host, hs, ws);
        forward(Bn, false);
      });
    } else {
      HCK(hipGraphCreate(&gr, 0));
      try {
        // a captured op is a chain of kernel nodes: re-add them as kernel nodes of the
        // parent (chained, the first one on `deps`); anything else becomes a child graph
        auto addChild = [&](hipGraph_t sub, const std::vector<hipGraphNode_t>& deps) {
          size_t nn = 0;
          HCK(hipGraphGetNodes(sub, nullptr, &nn));
          hipGraphNode_t node = nullptr;
          if (nn > 0) {
            std::vector<hipGraphNode_t> sn(nn);
            HCK(hipGraphGetNodes(sub, sn.data(), &nn));
            bool allKernels = true;
            for (auto x : sn) {
              hipGraphNodeType ty;
              HCK(hipGraphNodeGetType(x, &ty));
              allKernels = allKernels && ty == hipGraphNodeTypeKernel;
            }
            if (allKernels) {
              // captured nodes come back in capture (= dependency) order for a single stream
              std::vector<hipGraphNode_t> d = deps;
              for (auto x : sn) {
                hipKernelNodeParams kp{};
                HCK(hipGraphKernelNodeGetParams(x, &kp));
                HCK(hipGraphAddKernelNode(&node, gr, d.data(), d.size(), &kp));
                d.assign(1, node);
              }
            } else {
              HCK(hipGraphAddChildGraphNode(&node, gr, deps.data(), deps.size(), sub));
            }
          }
          HCK(hipGraphDestroy(sub));
          return node;
        };
        hipGraphNode_t pre = nullptr;
        if (frames) pre = addChild(captureOne([&] { preprocessFrames(Bn, *frames, host, hs, ws); }), {});
        const int n = (int)ops.size();
        const int inBuf = g.tens[0].buf;
        std::vector<hipGraphNode_t> node(n, nullptr);
        std::vector<char> hasSucc(n, 0);
        for (int k = 0; k < n; k++) {
          if (ops[k].chain < 0 || acc[k].empty()) continue;
          std::vector<hipGraphNode_t> deps;
          for (int d : dagDeps[k])
            if (node[d]) { deps.push_back(node[d]); hasSucc[d] = 1; }
          bool readsInput = false;
          for (const Acc& x : acc[k]) readsInput = readsInput || x.buf == inBuf;
          if (pre && (readsInput || deps.empty())) deps.push_back(pre);
          node[k] = addChild(captureOne([&] { runOp(k, Bn); }), deps);
        }
        std::vector<hipGraphNode_t> sinks;
        for (int k = 0; k < n; k++)
          if (node[k] && !hasSucc[k]) sinks.push_back(node[k]);
        if (sinks.empty() && pre) sinks.push_back(pre);
        addChild(captureOne([&] { post(Bn); }), sinks);
      } catch (...) {
        (void)hipGraphDestroy(gr);
        throw;
      }
    }
    hipGraphExec_t ex;
    HCK(hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0));
    HCK(hipGraphDestroy(gr));
    return ex;
  }

  void buildGraphs() {
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    graphs.assign(B, nullptr);
    execMs.assign(B, 0.f);
    for (int Bn = 1; Bn <= B; Bn++) {
      graphs[Bn - 1] = capture(Bn, nullptr, nullptr, nullptr, nullptr);
      for (int i = 0; i < 3; i++) HCK(hipGraphLaunch(graphs[Bn - 1], st));
      HCK(hipStreamSynchronize(st));
      HCK(hipEventRecord(e0, st));
      for (int i = 0; i < 10; i++) HCK(hipGraphLaunch(graphs[Bn - 1], st));
      HCK(hipEventRecord(e1, st));
      HCK(hipEventSynchronize(e1));
      float ms = 0.f;
      HCK(hipEventElapsedTime(&ms, e0, e1));
      execMs[Bn - 1] = ms / 10.f;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }

  SlotGeom geom(int sh, int sw) const {
    const BufDesc& ib = g.bufs[g.tens[0].buf];
    SlotGeom sg;
    sg.scale = std::min((float)ib.H / sh, (float)ib.W / sw);
    int nh = (int)roundf(sh * sg.scale), nw = (int)roundf(sw * sg.scale);
    sg.top = (ib.H - nh) / 2;
    sg.left = (ib.W - nw) / 2;
    return sg;
  }

  // The frame graph variant for the next frame: the one-block NMS while every slot of the
  // previous frame (the last results fetched to pinned memory; zeros before the first) had at
  // most NMS_BLOCK_MAX candidates, else the multi-block pipeline.
  bool sparsePrev() const {
    for (int s = 0; s < frameB; s++)
      if (h_rawcnt[s] > NMS_BLOCK_MAX) return false;
    return true;
  }
  hipGraphExec_t frameExec() const {
    return frameGraphBlock && sparsePrev() ? frameGraphBlock : frameGraph;
  }

  void run(int Bn) {
    if (Bn < 1 || Bn > B) throw Failure(fmt("batch %d outside 1..%d", Bn, B));
    if (!graphs.empty() && graphs[Bn - 1])
      HCK(hipGraphLaunch(graphs[Bn - 1], st));
    else
      forward(Bn);
  }
};

}  // namespace yolo

using yolo::Engine;
using yolo::Failure;

namespace {

void setErr(char* err, int errlen, const char* msg) {
  if (err && errlen > 0) {
    strncpy(err, msg, errlen - 1);
    err[errlen - 1] = 0;
  }
}

Engine* create(const char* dir, int maxB, int flags) {
  auto* e = new Engine();
  e->nmsBlock = (flags & YOLO_NMS_BLOCK) != 0;
  try {
    e->load(dir, maxB, !(flags & YOLO_NOFUSE));
    if (flags & YOLO_BRANCHES) {
      e->planStreams();
      e->createStreams();
    }
    if (!(flags & YOLO_NOTUNE)) e->autotune();
    // grouped launches for the single-stream plan (the DAG and side-stream plans keep one op
    // per launch); the group tuning may move ops off split-K, so splits are assigned after it
    e->planUnits(!(flags & (YOLO_NOTUNE | YOLO_DAGGRAPH | YOLO_BRANCHES | YOLO_NOGROUP)));
    if (flags & (YOLO_DAGGRAPH | YOLO_BRANCHES | YOLO_NOGROUP)) {
      e->units.clear();
      for (int k = 0; k < (int)e->ops.size(); k++) e->units.push_back({{k}, 0});
    }
    e->assignSplits();
    if (flags & YOLO_DAGGRAPH) e->planDag();
    if (!(flags & YOLO_NOGRAPH)) e->buildGraphs();
  } catch (...) {
    delete e;
    throw;
  }
  return e;
}

Engine* E(void* h) { return static_cast<Engine*>(h); }

template <typename F>
int guarded(F f) {
  try {
    return f();
  } catch (const std::exception& ex) {
    fprintf(stderr, "yolo: %s\n", ex.what());
    return -1;
  }
}

void fatal(const std::exception& ex) {
  fprintf(stderr, "yolo: %s\n", ex.what());
  exit(1);
}

}  // namespace

extern "C" {

void* yolo_create(const char* model_dir, int max_batch) {
  try {
    Engine* e = create(model_dir, max_batch, 0);
    printf("engine ready: B=1..%d, exec %.3f..%.3f ms\n", max_batch, e->execMs[0], e->execMs[max_batch - 1]);
    return e;
  } catch (const std::exception& ex) {
    fatal(ex);
  }
  return nullptr;
}

void* yolo_create_ex(const char* model_dir, int max_batch, int flags, char* err, int errlen) {
  try {
    return create(model_dir, max_batch, flags);
  } catch (const std::exception& ex) {
    setErr(err, errlen, ex.what());
    return nullptr;
  }
}

void yolo_destroy(void* h) {
  if (!h) return;
  (void)hipStreamSynchronize(E(h)->st);
  delete E(h);
}

int yolo_graph_check(const char* model_dir, char* err, int errlen) {
  try {
    yolo::GraphDesc g;
    std::string msg;
    if (!yolo::parseGraph(model_dir, g, msg) || !yolo::validateGraph(g, msg)) {
      setErr(err, errlen, msg.c_str());
      return -1;
    }
    return (int)g.ops.size();
  } catch (const std::exception& ex) {
    setErr(err, errlen, ex.what());
    return -1;
  }
}

int yolo_task(void* h) { return E(h)->g.seg ? 3 : (E(h)->g.obb ? 1 : (E(h)->g.cls ? 2 : 0)); }

float yolo_exec_ms(void* h, int B) {
  Engine* e = E(h);
  return (B >= 1 && B <= (int)e->execMs.size()) ? e->execMs[B - 1] : -1.f;
}

hipStream_t yolo_stream(void* h) { return E(h)->st; }

void yolo_preprocess(void* h, const unsigned char* dev_bgr, int height, int width, int slot) {
  Engine* e = E(h);
  try {
    if (slot < 0 || slot >= e->B) throw Failure("slot out of range");
    if (e->g.bufs[e->g.tens[0].buf].C != 3) throw Failure("letterbox needs a 3-channel input tensor");
    yolo::SlotGeom sg = e->geom(height, width);
    e->slots[slot] = sg;
    const yolo::BufDesc& ib = e->g.bufs[e->g.tens[0].buf];
    int nh = (int)roundf(height * sg.scale), nw = (int)roundf(width * sg.scale);
    yolo::launchPreprocess(dev_bgr, height, width, e->bufp[e->g.tens[0].buf] + (size_t)slot * ib.H * ib.W * 3,
                           ib.H, ib.W, sg.scale, sg.top, sg.left, nh, nw, e->st);
    HCK(hipGetLastError());
  } catch (const std::exception& ex) {
    fatal(ex);
  }
}

void yolo_run(void* h, int B) {
  try {
    E(h)->run(B);
    HCK(hipStreamSynchronize(E(h)->st));
  } catch (const std::exception& ex) {
    fatal(ex);
  }
}

void yolo_run_async(void* h, int B) {
  try {
    E(h)->run(B);
  } catch (const std::exception& ex) {
    fatal(ex);
  }
}

void yolo_sync(void* h) {
  try {
    HCK(hipStreamSynchronize(E(h)->st));
  } catch (const std::exception& ex) {
    fatal(ex);
  }
}

int yolo_get(void* h, int slot, YoloDet* out, int cap) {
  Engine* e = E(h);
  if (slot < 0 || slot >= e->B || e->g.obb) return 0;   // OBB records: yolo_get_obb
  const yolo::SlotGeom& sm = e->slots[slot];
  int cnt = std::min(e->h_cnt[slot], cap);
  for (int i = 0; i < cnt; i++) {
    const float* d = e->h_out + ((size_t)slot * yolo::MAX_OUT + i) * 6;
    out[i] = YoloDet{(d[0] - sm.left) / sm.scale, (d[1] - sm.top) / sm.scale, (d[2] - sm.left) / sm.scale,
                     (d[3] - sm.top) / sm.scale, d[4], (int)d[5]};
  }
  return cnt;
}

int yolo_get_batch(void* h, int B, YoloDet* out, int cap, int* counts) {
  Engine* e = E(h);
  if (B < 1 || B > e->B || cap < 0) return 0;
  int total = 0;
  for (int s = 0; s < B; s++) total += counts[s] = yolo_get(h, s, out + (size_t)s * cap, cap);
  return total;
}

static_assert(YOLO_PIXEL_BGR == yolo::PIXEL_BGR && YOLO_PIXEL_RGBX == yolo::PIXEL_RGBX, "pixel layouts");

int yolo_stage_frames(void* h, int B, const unsigned char* const* host, const int* heights, const int* widths,
                      int format, int first_slot) {
  return guarded([&] {
    Engine* e = E(h);
    if (B < 1 || first_slot < 0 || first_slot + B > e->B || !host || !heights || !widths ||
        (format != YOLO_PIXEL_BGR && format != YOLO_PIXEL_RGBX))
      return -1;
    e->checkFrameInput();
    for (int s = 0; s < B; s++)
      if (!host[s] || heights[s] <= 0 || widths[s] <= 0) return -1;
    e->waitDecoded();   // a decode may still be writing these slots' staging frames
    std::vector<std::pair<const uint8_t*, yolo::SlotGeom>> frames;
    for (int s = 0; s < B; s++) {
      e->forgetDecoded(first_slot + s);
      uint8_t* dev = e->stageBuffer(first_slot + s, (size_t)heights[s] * widths[s] * yolo::pixelBytes(format));
      const yolo::SlotGeom sg = e->geom(heights[s], widths[s]);
      if (!e->g.cls) e->slots[first_slot + s] = sg;
      frames.push_back({dev, sg});
    }
    e->preprocessFrames(B, frames, host, heights, widths, format, first_slot);
    HCK(hipGetLastError());
    return 0;
  });
}

namespace {

// What one batch decode can hold: the IDCT addresses blocks with 32-bit indices and the
// sample planes with 32-bit byte offsets.  admit() adds a stream if it still fits.
struct JpegBatchBudget {
  size_t blocks = 0, samples = 0;
  bool admit(const yolo::jpeg::Header& H) {
    size_t s = samples;
    for (int c = 0; c < H.nc; c++) s = (s + (size_t)H.comp[c].bw * H.comp[c].bh * 64 + 255) & ~(size_t)255;
    const size_t b = blocks + H.blocks();
    if (b >= (size_t)1 << 31 || s >= (size_t)1 << 32) return false;
    blocks = b;
    samples = s;
    return true;
  }
};

// Pinned buffers for the coefficients of yolo_jpeg_submit tickets, process-wide: a buffer
// goes back to the free list once the copy that read it has run (its event has completed).
// The free list keeps at most kKeepBytes in buffers of at most kKeepOne each; others are
// freed, so a burst of large frames does not leave gigabytes pinned.
struct CoefPool {
  static constexpr size_t kKeepOne = (size_t)64 << 20;
  static constexpr size_t kKeepBytes = (size_t)512 << 20;
  std::mutex mu;
  std::multimap<size_t, int16_t*> free;
  size_t freeBytes = 0;
  std::vector<std::pair<hipEvent_t, std::vector<std::pair<size_t, int16_t*>>>> retiring;

  void putLocked(size_t cap, int16_t* p) {
    if (cap > kKeepOne || freeBytes + cap > kKeepBytes) {
      (void)hipHostFree(p);
      return;
    }
    try {
      free.emplace(cap, p);
    } catch (...) {   // no memory for the list entry: give the buffer back instead
      (void)hipHostFree(p);
      return;
    }
    freeBytes += cap;
  }
  void reclaimLocked() {
    for (auto it = retiring.begin(); it != retiring.end();) {
      if (hipEventQuery(it->first) == hipSuccess) {
        for (auto& b : it->second) putLocked(b.first, b.second);
        (void)hipEventDestroy(it->first);
        it = retiring.erase(it);
      } else {
        ++it;
      }
    }
  }
  std::pair<size_t, int16_t*> take(size_t bytes) {
    {
      std::lock_guard<std::mutex> lk(mu);
      reclaimLocked();
      auto it = free.lower_bound(bytes);
      if (it != free.end() && it->first <= bytes * 2) {
        auto b = *it;
        free.erase(it);
        freeBytes -= b.first;
        return b;
      }
    }
    const size_t cap = std::max(bytes, (size_t)1 << 20);
    int16_t* p = nullptr;
    HCK(hipHostMalloc((void**)&p, cap, 0));
    return {cap, p};
  }
  void give(size_t cap, int16_t* p) {
    std::lock_guard<std::mutex> lk(mu);
    putLocked(cap, p);
  }
  void retire(hipEvent_t ev, std::vector<std::pair<size_t, int16_t*>> bufs) {
    std::lock_guard<std::mutex> lk(mu);
    retiring.emplace_back(ev, std::move(bufs));
  }
};

CoefPool& coefPool() {
  static CoefPool* p = new CoefPool;   // process lifetime (pinned memory is freed at exit)
  return *p;
}

}  // namespace

// A JPEG stream being entropy-decoded on a decoder thread (yolo_jpeg_submit).
struct JpegTicket {
  std::vector<uint8_t> data;
  yolo::jpeg::Header hd;
  size_t cap = 0;
  int16_t* coef = nullptr;   // pinned
  std::mutex mu;
  std::condition_variable cv;
  bool done = false, ok = false;

  void wait() {
    std::unique_lock<std::mutex> lk(mu);
    cv.wait(lk, [&] { return done; });
  }
};

// The GPU half of a batch decode.  Streams i with status[i] == YOLO_JPEG_STAGED have headers
// hd[i] and quantised coefficients at coef[i] (pinned host memory); the descriptors are written
// at S.host + descOff.  Streams past what one batch can hold (JpegBatchBudget) are set to
// YOLO_JPEG_UNSUPPORTED.  Copies coefficients and descriptors to the device, runs the IDCT and
// colour kernels into the slots' staging frames, records which slots hold a decoded frame and
// records S.copied after the copies.  Returns the number of streams converted.
int yolo::Engine::convertDecoded(int Bn, int firstSlot, const std::vector<jpeg::Header>& hd,
                           const std::vector<const int16_t*>& coef, int* status, JpegStage& S,
                           size_t descOff) {
  ensureDecodeStream();
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  {
    JpegBatchBudget budget;
    for (int i = 0; i < Bn; i++)
      if (status[i] == YOLO_JPEG_STAGED && !budget.admit(hd[i])) status[i] = YOLO_JPEG_UNSUPPORTED;
  }
  std::vector<size_t> block0(Bn, 0);
  size_t blocks = 0;
  bool contiguous = true;
  const int16_t* base = nullptr;
  for (int i = 0; i < Bn; i++) {
    if (status[i] != YOLO_JPEG_STAGED) continue;
    if (!base) base = coef[i] - blocks * 64;
    contiguous = contiguous && coef[i] == base + blocks * 64;
    block0[i] = blocks;
    blocks += hd[i].blocks();
  }
  const size_t coefBytes = blocks * 64 * sizeof(int16_t);
  const size_t planeBytes = up((size_t)3 * Bn * sizeof(JpegPlane));
  const size_t descBytes = planeBytes + (size_t)Bn * sizeof(JpegFrame);
  auto* planes = reinterpret_cast<JpegPlane*>(S.host + descOff);
  auto* frames = reinterpret_cast<JpegFrame*>(S.host + descOff + planeBytes);
  int np = 0, nf = 0, maxPix = 0;
  size_t sampleBytes = 0;
  for (int i = 0; i < Bn; i++) {
    if (status[i] != YOLO_JPEG_STAGED) continue;
    const jpeg::Header& H = hd[i];
    JpegFrame& F = frames[nf++];
    std::memset(&F, 0, sizeof F);
    F.dst = stageBuffer(firstSlot + i, (size_t)H.H * H.W * 4);
    F.H = H.H;
    F.W = H.W;
    F.nc = H.nc;
    size_t b0 = block0[i];
    for (int c = 0; c < H.nc; c++) {
      const jpeg::Comp& k = H.comp[c];
      JpegPlane& P = planes[np++];
      P.block0 = (uint32_t)b0;
      P.bw = (uint16_t)k.bw;
      P.bh = (uint16_t)k.bh;
      P.out = (uint32_t)sampleBytes;
      P.pad = 0;
      std::memcpy(P.q, H.q[k.tq], sizeof P.q);
      F.plane[c] = P.out;
      F.stride[c] = k.bw * 8;
      F.cw[c] = k.cw;
      F.ch[c] = k.ch;
      F.fh[c] = k.fh;
      F.fv[c] = k.fv;
      b0 += (size_t)k.bw * k.bh;
      sampleBytes = up(sampleBytes + (size_t)k.bw * k.bh * 64);
    }
    maxPix = std::max(maxPix, H.H * H.W);
  }
  if ((int)jpegH.size() < B) {
    jpegH.resize(B, 0);
    jpegW.resize(B, 0);
  }
  for (int i = 0; i < Bn; i++) {
    const bool ok = status[i] == YOLO_JPEG_STAGED;
    jpegH[firstSlot + i] = ok ? hd[i].H : 0;
    jpegW[firstSlot + i] = ok ? hd[i].W : 0;
  }
  if (nf == 0) return 0;
  const size_t descDev = up(coefBytes);
  growDevice(jpegDev, jpegDevCap, descDev + descBytes);
  growDevice(jpegSamples, jpegSamplesCap, sampleBytes);
  hipStream_t ds = decodeSt;
  if (contiguous) {
    HCK(hipMemcpyAsync(jpegDev, base, coefBytes, hipMemcpyHostToDevice, ds));
  } else {
    for (int i = 0; i < Bn; i++)
      if (status[i] == YOLO_JPEG_STAGED)
        HCK(hipMemcpyAsync(jpegDev + block0[i] * 64 * sizeof(int16_t), coef[i], hd[i].blocks() * 64 * sizeof(int16_t),
                           hipMemcpyHostToDevice, ds));
  }
  HCK(hipMemcpyAsync(jpegDev + descDev, S.host + descOff, descBytes, hipMemcpyHostToDevice, ds));
  HCK(hipEventRecord(S.copied, ds));
  S.pending = true;
  launchJpegIdct(reinterpret_cast<const int16_t*>(jpegDev), reinterpret_cast<const JpegPlane*>(jpegDev + descDev), np,
                 (int)blocks, jpegSamples, ds);
  // the colour kernel writes the staging frames: after the last letterbox read them
  HCK(hipStreamWaitEvent(ds, readDone, 0));
  launchJpegColor(jpegSamples, reinterpret_cast<const JpegFrame*>(jpegDev + descDev + planeBytes), nf, maxPix, ds);
  HCK(hipEventRecord(decodeDone, ds));
  decodePending = true;
  HCK(hipGetLastError());
  return nf;
}

// The next pinned staging area with at least `bytes`, once its previous copy has run.
yolo::Engine::JpegStage& yolo::Engine::nextStage(size_t bytes) {
  JpegStage& S = jpegStage[jpegNext];
  jpegNext ^= 1;
  if (S.pending) HCK(hipEventSynchronize(S.copied));
  S.pending = false;
  if (S.cap < bytes) {
    if (S.host) HCK(hipHostFree(S.host));
    S.host = nullptr;
    S.cap = 0;
    const size_t want = std::max(bytes, (size_t)1 << 20);
    HCK(hipHostMalloc((void**)&S.host, want, 0));
    S.cap = want;
  }
  if (!S.copied) HCK(hipEventCreateWithFlags(&S.copied, hipEventDisableTiming));
  return S;
}

int yolo_decode_jpeg(void* h, int B, const unsigned char* const* data, const size_t* sizes, int first_slot,
                     int* heights, int* widths, int* status) {
  return guarded([&] {
    Engine* e = E(h);
    if (B < 1 || first_slot < 0 || first_slot + B > e->B || !data || !sizes || !status) return -1;
    e->checkFrameInput();
    namespace J = yolo::jpeg;
    std::vector<J::Header> hd(B);
    std::vector<size_t> block0(B, 0);
    size_t blocks = 0;
    JpegBatchBudget budget;
    for (int i = 0; i < B; i++) {
      int r = data[i] ? J::parse(data[i], sizes[i], hd[i]) : J::INVALID;
      if (r == J::OK && !budget.admit(hd[i])) r = J::UNSUPPORTED;   // past what one batch holds
      status[i] = r == J::OK ? YOLO_JPEG_STAGED : r == J::UNSUPPORTED ? YOLO_JPEG_UNSUPPORTED : YOLO_JPEG_INVALID;
      if (heights) heights[i] = r == J::OK ? hd[i].H : 0;
      if (widths) widths[i] = r == J::OK ? hd[i].W : 0;
      if (r == J::OK) {
        block0[i] = blocks;
        blocks += hd[i].blocks();
      }
    }
    // pinned staging: [coefficients][descriptors]
    const size_t descOff = (blocks * 64 * sizeof(int16_t) + 255) & ~(size_t)255;
    Engine::JpegStage& S = e->nextStage(descOff + 3 * (size_t)B * sizeof(yolo::JpegPlane) + 256 +
                                        (size_t)B * sizeof(yolo::JpegFrame));
    int16_t* coef = reinterpret_cast<int16_t*>(S.host);
    J::parallelFor(B, [&](int i) {
      if (status[i] == YOLO_JPEG_STAGED && !J::decode(data[i], sizes[i], hd[i], coef + block0[i] * 64))
        status[i] = YOLO_JPEG_INVALID;
    });
    std::vector<const int16_t*> src(B, nullptr);
    for (int i = 0; i < B; i++) src[i] = coef + block0[i] * 64;
    return B - e->convertDecoded(B, first_slot, hd, src, status, S, descOff);
  });
}

void* yolo_jpeg_submit(const unsigned char* data, size_t size) {
  if (!data) return nullptr;
  try {
    auto t = std::make_unique<JpegTicket>();
    if (yolo::jpeg::parse(data, size, t->hd) != yolo::jpeg::OK) return nullptr;
    t->data.assign(data, data + size);
    auto buf = coefPool().take(t->hd.blocks() * 64 * sizeof(int16_t));
    t->cap = buf.first;
    t->coef = buf.second;
    JpegTicket* tp = t.get();
    try {
      yolo::jpeg::runAsync([tp] {
        const bool ok = yolo::jpeg::decode(tp->data.data(), tp->data.size(), tp->hd, tp->coef);
        std::lock_guard<std::mutex> lk(tp->mu);
        tp->ok = ok;
        tp->done = true;
        tp->cv.notify_all();
      });
    } catch (...) {   // not queued: the ticket (freed by t) never reaches the decoder
      coefPool().give(tp->cap, tp->coef);
      throw;
    }
    return t.release();
  } catch (const std::exception& ex) {
    std::fprintf(stderr, "[yolo] yolo_jpeg_submit: %s\n", ex.what());
    return nullptr;
  }
}

void yolo_jpeg_release(void* ticket) {
  auto* t = static_cast<JpegTicket*>(ticket);
  if (!t) return;
  t->wait();
  coefPool().give(t->cap, t->coef);   // never copied from
  delete t;
}

int yolo_decode_tickets(void* h, int B, void* const* tickets, int first_slot, int* heights, int* widths,
                        int* status) {
  if (!tickets || B < 1) return -1;
  std::vector<JpegTicket*> ts(B);
  for (int i = 0; i < B; i++) ts[i] = static_cast<JpegTicket*>(tickets[i]);
  bool copied = false;
  hipEvent_t ev = nullptr;
  const int r = guarded([&] {
    Engine* e = E(h);
    if (first_slot < 0 || first_slot + B > e->B || !status) return -1;
    e->checkFrameInput();
    std::vector<yolo::jpeg::Header> hd(B);
    std::vector<const int16_t*> src(B, nullptr);
    for (int i = 0; i < B; i++) {
      JpegTicket* t = ts[i];
      if (t) t->wait();
      status[i] = t && t->ok ? YOLO_JPEG_STAGED : YOLO_JPEG_INVALID;
      if (t) {
        hd[i] = t->hd;
        src[i] = t->coef;
      }
    }
    Engine::JpegStage& S = e->nextStage(3 * (size_t)B * sizeof(yolo::JpegPlane) + 256 + (size_t)B * sizeof(yolo::JpegFrame));
    const int nf = e->convertDecoded(B, first_slot, hd, src, status, S, 0);
    for (int i = 0; i < B; i++) {   // after convertDecoded: it may refuse streams past the batch budget
      if (heights) heights[i] = status[i] == YOLO_JPEG_STAGED ? hd[i].H : 0;
      if (widths) widths[i] = status[i] == YOLO_JPEG_STAGED ? hd[i].W : 0;
    }
    if (nf > 0) {
      HCK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
      HCK(hipEventRecord(ev, e->decodeSt));
      copied = true;
    }
    return B - nf;
  });
  // the tickets are consumed: buffers a copy read wait for its event, the others are free now
  // (after a failure, once the stream has passed whatever was queued)
  if (r < 0 && h) {
    (void)hipStreamSynchronize(E(h)->st);
    if (E(h)->decodeSt) (void)hipStreamSynchronize(E(h)->decodeSt);
  }
  std::vector<std::pair<size_t, int16_t*>> used;
  for (int i = 0; i < B; i++) {
    JpegTicket* t = ts[i];
    if (!t) continue;
    t->wait();
    if (r >= 0 && copied && status[i] == YOLO_JPEG_STAGED) used.emplace_back(t->cap, t->coef);
    else coefPool().give(t->cap, t->coef);
    delete t;
  }
  if (!used.empty()) coefPool().retire(ev, std::move(used));
  else if (ev) (void)hipEventDestroy(ev);
  return r;
}

int yolo_letterbox_decoded(void* h, int B, int first_slot) {
  return guarded([&] {
    Engine* e = E(h);
    if (B < 1 || first_slot < 0 || first_slot + B > e->B) return -1;
    e->checkFrameInput();
    std::vector<Engine::Staged> v;
    for (int s = first_slot; s < first_slot + B; s++) {
      if (s >= (int)e->jpegH.size() || e->jpegH[s] <= 0) continue;
      const yolo::SlotGeom sg = e->geom(e->jpegH[s], e->jpegW[s]);
      if (!e->g.cls) e->slots[s] = sg;
      v.push_back(Engine::Staged{s, e->stageDev[s], e->jpegH[s], e->jpegW[s], sg});
    }
    if (!v.empty()) {
      e->waitDecoded();
      e->preprocessStaged(v, yolo::PIXEL_RGBX);
    }
    HCK(hipGetLastError());
    return (int)v.size();
  });
}

int yolo_stage_jpeg(void* h, int B, const unsigned char* const* data, const size_t* sizes, int first_slot,
                    int* heights, int* widths, int* status) {
  const int failed = yolo_decode_jpeg(h, B, data, sizes, first_slot, heights, widths, status);
  if (failed < 0 || failed == B) return failed;
  return yolo_letterbox_decoded(h, B, first_slot) < 0 ? -1 : failed;
}

void yolo_preprocess_cls(void* h, const unsigned char* dev_bgr, int height, int width, int slot) {
  Engine* e = E(h);
  try {
    if (slot < 0 || slot >= e->B) throw Failure("slot out of range");
    if (e->g.bufs[e->g.tens[0].buf].C != 3) throw Failure("classify preprocess needs a 3-channel input tensor");
    const yolo::BufDesc& ib = e->g.bufs[e->g.tens[0].buf];
    if (ib.H != ib.W) throw Failure("classify preprocess needs a square input");
    const yolo::ClsGeom cg = yolo::clsGeom(ib.H, height, width);
    yolo::launchPreprocessCls(dev_bgr, height, width, e->bufp[e->g.tens[0].buf] + (size_t)slot * ib.H * ib.W * 3,
                              ib.H, cg.rh, cg.rw, cg.top, cg.left, yolo::PIXEL_BGR, e->st);
    HCK(hipGetLastError());
  } catch (const std::exception& ex) {
    fatal(ex);
  }
}

// Top-k class ids and probabilities of a slot from the pinned fp16 probabilities: insertion
// into k ranked slots with a strict comparison, so among equal probabilities the lower class
// id ranks first (engine/engine.cu:1593-1606).  Returns min(k, nc); 0 for non-classify
// handles (engine/engine.cu:1768-1773).
int yolo_get_cls(void* h, int slot, int* ids, float* probs, int k) {
  Engine* e = E(h);
  if (!e->g.cls || slot < 0 || slot >= e->B || k <= 0) return 0;
  k = std::min(k, e->g.nc);
  for (int i = 0; i < k; i++) { ids[i] = -1; probs[i] = -1.f; }
  const yolo::f16* p = e->h_probs + (size_t)slot * e->g.nc;
  for (int c = 0; c < e->g.nc; c++) {
    const float v = (float)p[c];
    for (int i = 0; i < k; i++) {
      if (v > probs[i]) {
        for (int j = k - 1; j > i; j--) { probs[j] = probs[j - 1]; ids[j] = ids[j - 1]; }
        probs[i] = v;
        ids[i] = c;
        break;
      }
    }
  }
  return k;
}

void yolo_slot_geom(void* h, int slot, float* scale, int* top, int* left) {
  Engine* e = E(h);
  if (slot < 0 || slot >= e->B) return;
  *scale = e->slots[slot].scale;
  *top = e->slots[slot].top;
  *left = e->slots[slot].left;
}

// Rotated boxes in original-image coordinates: centre un-padded, centre and size divided by
// the letterbox scale, angle unchanged, no clipping (engine/engine.cu:1783-1794).
int yolo_get_obb(void* h, int slot, YoloObbDet* out, int cap) {
  Engine* e = E(h);
  if (slot < 0 || slot >= e->B || !e->g.obb) return 0;
  const yolo::SlotGeom& sm = e->slots[slot];
  int cnt = std::min(e->h_cnt[slot], cap);
  for (int i = 0; i < cnt; i++) {
    const float* d = e->h_out + ((size_t)slot * yolo::MAX_OUT + i) * 7;
    out[i] = YoloObbDet{(d[0] - sm.left) / sm.scale, (d[1] - sm.top) / sm.scale, d[2] / sm.scale,
                        d[3] / sm.scale, d[6], d[4], (int)d[5]};
  }
  return cnt;
}

int yolo_get_obb_batch(void* h, int B, YoloObbDet* out, int cap, int* counts) {
  Engine* e = E(h);
  if (B < 1 || B > e->B || cap < 0) return 0;
  int total = 0;
  for (int s = 0; s < B; s++) total += counts[s] = yolo_get_obb(h, s, out + (size_t)s * cap, cap);
  return total;
}

void yolo_mask_dim(void* h, int* ph, int* pw) {
  Engine* e = E(h);
  if (e->g.protoTen < 0) { *ph = *pw = 0; return; }
  const yolo::BufDesc& b = e->g.bufs[e->g.tens[e->g.protoTen].buf];
  *ph = b.H;
  *pw = b.W;
}

int yolo_get_mask(void* h, int slot, int det, unsigned char* out) {
  Engine* e = E(h);
  if (e->g.protoTen < 0 || slot < 0 || slot >= e->B || det < 0 || det >= e->h_cnt[slot]) return -1;
  const yolo::BufDesc& b = e->g.bufs[e->g.tens[e->g.protoTen].buf];
  size_t sz = (size_t)b.H * b.W;
  return hipMemcpy(out, e->masks + ((size_t)slot * yolo::MAX_OUT + det) * sz, sz, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}

int yolo_get_masks(void* h, int slot, int first, int n, unsigned char* out) {
  Engine* e = E(h);
  if (e->g.protoTen < 0 || slot < 0 || slot >= e->B || first < 0 || n < 1 || first + n > e->h_cnt[slot] || !out)
    return -1;
  const yolo::BufDesc& b = e->g.bufs[e->g.tens[e->g.protoTen].buf];
  const size_t sz = (size_t)b.H * b.W;
  return hipMemcpy(out, e->masks + ((size_t)slot * yolo::MAX_OUT + first) * sz, sz * n, hipMemcpyDeviceToHost) ==
                 hipSuccess
             ? 0
             : -1;
}

int yolo_set_thresholds(void* h, float conf, float iou, int max_det) {
  Engine* e = E(h);
  if (max_det < 0 || max_det > yolo::MAX_OUT || !(iou >= 0.f) || !(conf >= 0.f)) return -1;
  e->hparams = yolo::PostParams{conf, iou, max_det, 0};
  return hipMemcpy(e->params, &e->hparams, sizeof(yolo::PostParams), hipMemcpyHostToDevice) == hipSuccess ? 0 : -1;
}

int yolo_raw_count(void* h, int slot) {
  Engine* e = E(h);
  return (slot >= 0 && slot < e->B) ? e->h_rawcnt[slot] : -1;
}

int yolo_num_ops(void* h) { return (int)E(h)->ops.size(); }

int yolo_op_info(void* h, int k, int* info) {
  Engine* e = E(h);
  if (k < 0 || k >= (int)e->ops.size()) return -1;
  const yolo::OpDesc& op = e->ops[k];
  int v[9] = {op.kind, op.a, op.b, op.out, op.k, op.s, op.g, op.Cin, op.Cout};
  memcpy(info, v, sizeof v);
  return 0;
}

int yolo_num_tensors(void* h) { return (int)E(h)->g.tens.size(); }

int yolo_tensor_shape(void* h, int t, int* hwc) {
  Engine* e = E(h);
  if (t < 0 || t >= (int)e->g.tens.size()) return -1;
  yolo::View v = e->view(t);
  hwc[0] = v.H;
  hwc[1] = v.W;
  hwc[2] = v.C;
  return 0;
}

// Tensor reads and writes for the parity harness.  A view is n*H*W pixel rows of C halves at
// a row stride of s halves; a 2-D copy with one row per pixel costs microseconds per row on
// this runtime (seconds for a batch-32 80x80 tensor), so the span from the first row to the
// end of the last is moved with one 1-D copy and the rows are gathered or scattered on the
// host (a write reads the span first, so channels outside the view are left as they are).
namespace {
struct TensorSpan {
  yolo::f16* dev;   // first element of the view's first row
  size_t rows, C, s, bytes;
};
TensorSpan tensorSpan(const yolo::View& v, int first, int n) {
  const size_t img = (size_t)v.H * v.W * v.s, rows = (size_t)n * v.H * v.W;
  return {v.p + first * img + v.o, rows, (size_t)v.C, (size_t)v.s, ((rows - 1) * v.s + v.C) * sizeof(yolo::f16)};
}
}  // namespace

int yolo_read_tensor_slots(void* h, int t, int first, int n, void* host_f16) {
  return guarded([&] {
    Engine* e = E(h);
    if (t < 0 || t >= (int)e->g.tens.size() || first < 0 || n < 1 || first + n > e->B) return -1;
    const TensorSpan sp = tensorSpan(e->view(t), first, n);
    HCK(hipStreamSynchronize(e->st));
    if (sp.s == sp.C) {
      HCK(hipMemcpy(host_f16, sp.dev, sp.bytes, hipMemcpyDeviceToHost));
      return 0;
    }
    std::vector<yolo::f16> tmp(sp.bytes / sizeof(yolo::f16));
    HCK(hipMemcpy(tmp.data(), sp.dev, sp.bytes, hipMemcpyDeviceToHost));
    auto* out = static_cast<yolo::f16*>(host_f16);
    for (size_t r = 0; r < sp.rows; r++) std::memcpy(out + r * sp.C, tmp.data() + r * sp.s, sp.C * sizeof(yolo::f16));
    return 0;
  });
}

int yolo_write_tensor_slots(void* h, int t, int first, int n, const void* host_f16) {
  return guarded([&] {
    Engine* e = E(h);
    if (t < 0 || t >= (int)e->g.tens.size() || first < 0 || n < 1 || first + n > e->B) return -1;
    const TensorSpan sp = tensorSpan(e->view(t), first, n);
    HCK(hipStreamSynchronize(e->st));
    if (sp.s == sp.C) {
      HCK(hipMemcpy(sp.dev, host_f16, sp.bytes, hipMemcpyHostToDevice));
      return 0;
    }
    std::vector<yolo::f16> tmp(sp.bytes / sizeof(yolo::f16));
    HCK(hipMemcpy(tmp.data(), sp.dev, sp.bytes, hipMemcpyDeviceToHost));
    const auto* in = static_cast<const yolo::f16*>(host_f16);
    for (size_t r = 0; r < sp.rows; r++) std::memcpy(tmp.data() + r * sp.s, in + r * sp.C, sp.C * sizeof(yolo::f16));
    HCK(hipMemcpy(sp.dev, tmp.data(), sp.bytes, hipMemcpyHostToDevice));
    return 0;
  });
}

int yolo_read_tensor(void* h, int t, int B, void* host_f16) { return yolo_read_tensor_slots(h, t, 0, B, host_f16); }

int yolo_write_tensor(void* h, int t, int B, const void* host_f16) {
  return yolo_write_tensor_slots(h, t, 0, B, host_f16);
}

int yolo_run_op(void* h, int k, int B) {
  return guarded([&] {
    Engine* e = E(h);
    if (k < 0 || k >= (int)e->ops.size() || B < 1 || B > e->B) return -1;
    // ops run one at a time may repeat a decode without NMS in between: start its
    // candidate lists empty
    if (k == e->lastDecode) HCK(hipMemsetAsync(e->nmsCount, 0, (size_t)e->B * sizeof(int), e->st));
    e->runOp(k, B);
    HCK(hipGetLastError());
    HCK(hipStreamSynchronize(e->st));
    return 0;
  });
}

int yolo_run_post(void* h, int B) {
  return guarded([&] {
    Engine* e = E(h);
    if (B < 1 || B > e->B) return -1;
    e->post(B);
    HCK(hipGetLastError());
    HCK(hipStreamSynchronize(e->st));
    return 0;
  });
}

int yolo_op_config(void* h, int k) {
  Engine* e = E(h);
  if (k < 0 || k >= (int)e->ops.size()) return -1;
  const yolo::OpDesc& op = e->ops[k];
  if (op.kind != yolo::CONV || op.g != 1 || op.Cin == 3) return -1;
  if (op.cfg >= 0) return op.cfg;
  yolo::View y = e->view(op.out);
  return yolo::heuristicTile(e->B * y.H * y.W, op.Cout, op.k * op.k * op.Cin);
}

int yolo_set_op_config(void* h, int k, int cfg) {
  Engine* e = E(h);
  if (k < 0 || k >= (int)e->ops.size()) return -1;
  yolo::OpDesc& op = e->ops[k];
  if (op.kind != yolo::CONV || op.g != 1 || op.Cin == 3) return -1;
  if (yolo::specialConvCfg(cfg)) {
    yolo::View r{};
    if (op.b >= 0) r = e->view(op.b);
    const yolo::View* rp = op.b >= 0 ? &r : nullptr;
    if (!yolo::specialConvOk(cfg, e->view(op.a), e->view(op.out), rp, op.k, op.s, op.p)) return -1;
  } else if (cfg >= yolo::numTileConfigs()) {
    return -1;
  }
  op.cfg = cfg < 0 ? -1 : cfg;
  op.split = 1;                 // a different tile needs a different split workspace
  op.tail = -1;
  op.wsOff = op.cntOff = -1;
  return 0;
}

int yolo_op_tail(void* h, int k) {
  Engine* e = E(h);
  if (k < 0 || k >= (int)e->ops.size()) return -2;
  const yolo::OpDesc& op = e->ops[k];
  if (op.kind != yolo::CONV || op.g != 1 || op.Cin == 3) return -2;
  return op.tail;
}

int yolo_set_op_tail(void* h, int k, int tail) {
  Engine* e = E(h);
  if (k < 0 || k >= (int)e->ops.size()) return -1;
  yolo::OpDesc& op = e->ops[k];
  if (op.kind != yolo::CONV || op.g != 1 || op.Cin == 3 || yolo::specialConvCfg(op.cfg) || op.split != 1) return -1;
  if (tail < 0) {
    op.tail = -1;
    return 0;
  }
  const yolo::View y = e->view(op.out);
  const int M = e->B * y.H * y.W, K = op.k * op.k * op.Cin;
  const int cfg = op.cfg >= 0 ? op.cfg : yolo::heuristicTile(M, op.Cout, K);
  if (!yolo::tailOk(cfg, tail, op.k, op.s, op.p, op.Cin, M, op.Cout)) return -1;
  op.cfg = cfg;
  op.tail = tail;
  return 0;
}

int yolo_op_split(void* h, int k) {
  Engine* e = E(h);
  if (k < 0 || k >= (int)e->ops.size()) return -1;
  const yolo::OpDesc& op = e->ops[k];
  if (op.kind != yolo::CONV || op.g != 1 || op.Cin == 3) return -1;
  return op.split;
}

int yolo_set_op_split(void* h, int k, int splits) {
  return guarded([&] {
    Engine* e = E(h);
    if (k < 0 || k >= (int)e->ops.size()) return -1;
    yolo::OpDesc& op = e->ops[k];
    if (op.kind != yolo::CONV || op.g != 1 || op.Cin == 3) return -1;
    if (yolo::specialConvCfg(op.cfg)) return -1;   // not GEMM tiles
    bool captured = e->frameGraph != nullptr;
    for (auto ge : e->graphs) captured = captured || ge != nullptr;
    if (captured) return -1;    // captured graphs hold the current workspace pointers
    const yolo::View y = e->view(op.out);
    const int M = e->B * y.H * y.W, K = op.k * op.k * op.Cin;
    const int cfg = op.cfg >= 0 ? op.cfg : yolo::heuristicTile(M, op.Cout, K);
    if (splits == 0 || splits > yolo::MAX_SPLITS || splits < -yolo::MAX_SPLITS || !yolo::splitOk(cfg, K, splits))
      return -1;
    op.cfg = cfg;
    op.split = splits;
    if (splits != 1) op.tail = -1;
    e->assignSplits();
    return 0;
  });
}

int yolo_num_tile_configs(void) { return yolo::numTileConfigs(); }

int yolo_tile_config(int cfg, int* out) {
  if (cfg < 0 || cfg >= yolo::numTileConfigs()) return -1;
  const yolo::TileCfg& t = yolo::tileConfig(cfg);
  out[0] = t.BM;
  out[1] = t.BN;
  out[2] = t.WM;
  out[3] = t.WN;
  out[4] = t.BK;
  out[5] = t.NS;
  return 0;
}

int yolo_frame_graph(void* h, int B, const unsigned char* const* dev_bgr, const unsigned char* const* host_bgr,
                     const int* heights, const int* widths) {
  return guarded([&] {
    Engine* e = E(h);
    if (B < 1 || B > e->B) return -1;
    if (e->g.bufs[e->g.tens[0].buf].C != 3) throw Failure("letterbox needs a 3-channel input tensor");
    std::vector<std::pair<const uint8_t*, yolo::SlotGeom>> frames;
    for (int s = 0; s < B; s++) {
      if (!dev_bgr[s] || heights[s] <= 0 || widths[s] <= 0) return -1;
      frames.push_back({dev_bgr[s], e->geom(heights[s], widths[s])});
    }
    if (e->frameGraph) HCK(hipGraphExecDestroy(e->frameGraph));
    if (e->frameGraphBlock) HCK(hipGraphExecDestroy(e->frameGraphBlock));
    e->frameGraph = e->frameGraphBlock = nullptr;
    e->frameGraph = e->capture(B, &frames, host_bgr, heights, widths);
    if (e->nmsWork) {
      e->capBlock = true;
      try {
        e->frameGraphBlock = e->capture(B, &frames, host_bgr, heights, widths);
      } catch (...) {
        e->capBlock = false;
        throw;
      }
      e->capBlock = false;
    }
    e->frameB = B;
    e->frameSrc = frames;
    e->frameH.assign(heights, heights + B);
    e->frameW.assign(widths, widths + B);
    for (int s = 0; s < B; s++) e->slots[s] = frames[s].second;
    return 0;
  });
}

int yolo_frame_run(void* h) {
  return guarded([&] {
    Engine* e = E(h);
    if (!e->frameGraph) return -1;
    HCK(hipGraphLaunch(e->frameExec(), e->st));
    HCK(hipStreamSynchronize(e->st));
    return 0;
  });
}

int yolo_frame_launch(void* h) {
  return guarded([&] {
    Engine* e = E(h);
    if (!e->frameGraph) return -1;
    HCK(hipGraphLaunch(e->frameExec(), e->st));
    return 0;
  });
}

float yolo_time_graph(void* h, int which, int B, int iters) {
  float result = -1.f;
  guarded([&] {
    Engine* e = E(h);
    hipGraphExec_t ge = nullptr;
    if (which == 1) ge = e->frameGraph ? e->frameExec() : nullptr;
    else if (B >= 1 && B <= (int)e->graphs.size()) ge = e->graphs[B - 1];
    if (!ge || iters < 1) return -1;
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    HCK(hipEventRecord(e0, e->st));
    for (int i = 0; i < iters; i++) HCK(hipGraphLaunch(ge, e->st));
    HCK(hipEventRecord(e1, e->st));
    HCK(hipEventSynchronize(e1));
    float ms = 0.f;
    HCK(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    result = ms / iters;
    return 0;
  });
  return result;
}

int yolo_profile_ops(void* h, int B, int iters, float* ms) {
  return guarded([&] {
    Engine* e = E(h);
    if (B < 1 || B > e->B || iters < 1) return -1;
    const int n = (int)e->ops.size();
    std::vector<hipEvent_t> ev(n + 1);
    for (auto& x : ev) HCK(hipEventCreate(&x));
    std::vector<double> acc(n, 0.0);
    for (int it = 0; it < iters; it++) {
      HCK(hipMemsetAsync(e->nmsCount, 0, (size_t)e->B * sizeof(int), e->st));   // no NMS here
      HCK(hipEventRecord(ev[0], e->st));
      for (int k = 0; k < n; k++) {
        if (e->ops[k].chain >= 0) e->runOp(k, B);   // chain followers run inside the head
        HCK(hipEventRecord(ev[k + 1], e->st));
      }
      HCK(hipEventSynchronize(ev[n]));
      for (int k = 0; k < n; k++) {
        float t = 0.f;
        HCK(hipEventElapsedTime(&t, ev[k], ev[k + 1]));
        acc[k] += t;
      }
    }
    HCK(hipMemsetAsync(e->nmsCount, 0, (size_t)e->B * sizeof(int), e->st));
    for (auto& x : ev) hipEventDestroy(x);
    for (int k = 0; k < n; k++) ms[k] = (float)(acc[k] / iters);
    return 0;
  });
}

int yolo_profile_units(void* h, int B, int iters, int reps, float* ms) {
  return guarded([&] {
    Engine* e = E(h);
    if (B < 1 || B > e->B || iters < 1 || reps < 1) return -1;
    const int n = (int)e->ops.size();
    std::vector<double> acc(n, 0.0);
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    for (int it = 0; it < iters; it++)
      for (const auto& u : e->units) {
        const int k0 = u.ops[0];
        if (yolo::isDecode(e->ops[k0].kind) || e->ops[k0].chain < 0) continue;
        e->runUnit(u, B);   // warm: caches, clocks
        HCK(hipEventRecord(e0, e->st));
        for (int r = 0; r < reps; r++) e->runUnit(u, B);
        HCK(hipEventRecord(e1, e->st));
        HCK(hipEventSynchronize(e1));
        float t = 0.f;
        HCK(hipEventElapsedTime(&t, e0, e1));
        acc[*std::min_element(u.ops.begin(), u.ops.end())] += t / reps;   // the unit's first op
      }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    for (int k = 0; k < n; k++) ms[k] = (float)(acc[k] / iters);
    return 0;
  });
}

int yolo_num_units(void* h) { return (int)E(h)->units.size(); }

int yolo_run_unit(void* h, int u, int B) {
  return guarded([&] {
    Engine* e = E(h);
    if (u < 0 || u >= (int)e->units.size() || B < 1 || B > e->B) return -1;
    const int k0 = e->units[u].ops[0];
    if (yolo::isDecode(e->ops[k0].kind) || e->ops[k0].chain < 0) return 0;   // launched elsewhere
    e->runUnit(e->units[u], B);
    HCK(hipGetLastError());
    return 0;
  });
}

int yolo_marker(void* h) {
  return guarded([&] {
    yolo::launchMarker(E(h)->st);
    HCK(hipGetLastError());
    return 0;
  });
}

int yolo_spin_failures(void* h) {
  if (!h) return -1;
  return guarded([&] {
    HCK(hipStreamSynchronize(E(h)->st));
    return yolo::convSpinFailures();
  });
}

int yolo_op_unit(void* h, int k) {
  Engine* e = E(h);
  if (k < 0 || k >= (int)e->ops.size()) return -2;
  if (yolo::isDecode(e->ops[k].kind) || e->ops[k].chain < 0) return -1;
  for (int u = 0; u < (int)e->units.size(); u++)
    for (int j : e->units[u].ops)
      if (j == k) return u;
  return -1;
}

int yolo_profile_stages(void* h, int iters, float* ms) {
  return guarded([&] {
    Engine* e = E(h);
    if (!e->frameGraph || iters < 1 || e->g.cls || e->g.numAnchors == 0) return -1;
    const int Bn = e->frameB, n = (int)e->ops.size();
    hipEvent_t ev[7];
    for (auto& x : ev) HCK(hipEventCreate(&x));
    double acc[4] = {0, 0, 0, 0};
    HCK(hipMemsetAsync(e->nmsCount, 0, (size_t)e->B * sizeof(int), e->st));
    for (int it = 0; it < iters; it++) {
      HCK(hipEventRecord(ev[0], e->st));
      e->preprocessFrames(Bn, e->frameSrc, nullptr, e->frameH.data(), e->frameW.data());
      HCK(hipEventRecord(ev[1], e->st));
      for (int k = 0; k < n; k++) {
        if (e->ops[k].chain < 0) continue;
        if (k == e->lastDecode) HCK(hipEventRecord(ev[2], e->st));
        e->runOp(k, Bn);
        if (k == e->lastDecode) HCK(hipEventRecord(ev[3], e->st));
      }
      HCK(hipEventRecord(ev[4], e->st));
      // the NMS variant the frame graph would take for this frame
      const bool multi = e->nmsWork && !(e->frameGraphBlock && e->sparsePrev());
      if (e->g.obb && multi)
        yolo::launchNmsObbMulti(e->cand, e->nmsScratch, e->nmsCount, e->g.numAnchors, e->outdets, e->outidx,
                                e->outcnt, e->rawcnt, e->params, e->nmsWork, Bn, e->st);
      else if (e->g.obb)
        yolo::launchNmsObb(e->cand, e->nmsScratch, e->nmsCount, e->g.numAnchors, e->outdets, e->outidx, e->outcnt,
                           e->rawcnt, e->params, Bn, e->st);
      else if (multi)
        yolo::launchNmsMulti(e->cand, e->nmsScratch, e->nmsCount, e->g.numAnchors, e->cstride, e->outdets,
                             e->outidx, e->outcnt, e->rawcnt, e->params, e->nmsWork, Bn, e->st);
      else
        yolo::launchNms(e->cand, e->nmsScratch, e->nmsCount, e->g.numAnchors, e->cstride, e->outdets, e->outidx,
                        e->outcnt, e->rawcnt, e->params, Bn, e->st);
      HCK(hipEventRecord(ev[5], e->st));
      if (e->g.protoTen >= 0) {
        yolo::View pr = e->view(e->g.protoTen);
        const yolo::BufDesc& ib = e->g.bufs[e->g.tens[0].buf];
        yolo::launchMasks(pr, e->cand, e->cstride, e->g.numAnchors, e->g.nm, e->outidx, e->outcnt, e->outdets,
                          e->masks, (float)pr.W / ib.W, (float)pr.H / ib.H, Bn, e->st);
      }
      HCK(hipEventRecord(ev[6], e->st));
      HCK(hipEventSynchronize(ev[6]));
      float t;
      HCK(hipEventElapsedTime(&t, ev[0], ev[1])); acc[0] += t;
      HCK(hipEventElapsedTime(&t, ev[2], ev[3])); acc[1] += t;
      HCK(hipEventElapsedTime(&t, ev[4], ev[5])); acc[2] += t;
      HCK(hipEventElapsedTime(&t, ev[5], ev[6])); acc[3] += t;
    }
    for (auto& x : ev) (void)hipEventDestroy(x);
    for (int i = 0; i < 4; i++) ms[i] = (float)(acc[i] / iters);
    return 0;
  });
}

void* yolo_dev_alloc(size_t bytes) {
  void* p = nullptr;
  return hipMalloc(&p, bytes) == hipSuccess ? p : nullptr;
}

void yolo_dev_free(void* p) {
  if (p) (void)hipFree(p);
}

void* yolo_host_alloc(size_t bytes) {
  void* p = nullptr;
  return hipHostMalloc(&p, bytes, hipHostMallocDefault) == hipSuccess ? p : nullptr;
}

void yolo_host_free(void* p) {
  if (p) (void)hipHostFree(p);
}

int yolo_copy_h2d(void* h, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    HCK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, E(h)->st));
    HCK(hipStreamSynchronize(E(h)->st));
    return 0;
  });
}

int yolo_copy_d2h(void* h, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    HCK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, E(h)->st));
    HCK(hipStreamSynchronize(E(h)->st));
    return 0;
  });
}

}  // extern "C"
