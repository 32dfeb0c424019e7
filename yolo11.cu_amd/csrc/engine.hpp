// Internal declarations of the MI355X YOLO engine: graph description (host), device views
// and the kernel launchers every .hip file exports to the host runtime.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>
#include <vector>

namespace yolo {

typedef _Float16 f16;

// ------------------------------------------------------------------ graph (host side)
// Op kinds keep the reference's numbering (engine/engine.cu:33-34).
enum OpKind { CONV = 0, ADD, MAXPOOL5, UPSAMPLE2, COPYC, ATTN, DECODE, GAP, SOFTMAX, DECODEOBB,
              PS2, DECODESEG, MASKS };

inline bool isDecode(int kind) { return kind == DECODE || kind == DECODESEG || kind == DECODEOBB; }

struct BufDesc { int H, W, C; };
struct TenDesc { int buf, coff, C; };
struct OpDesc {
  int kind = 0;
  int a = -1, b = -1, out = -1;       // CONV: a = input, b = fused residual (-1 none)
  int k = 0, s = 0, p = 0, g = 0, act = 0, Cin = 0, Cout = 0;
  long woff = 0, boff = 0;
  int heads = 0, kd = 0, hd = 0;      // ATTN
  int stride = 0;                     // DECODE*
  int cfg = -1;                       // GEMM tile config (-1 = heuristic)
  int split = 1;                      // GEMM split-K factor (< -1: tail split, see conv.hip)
  int tail = -1;                      // GEMM tail retile config (-1 none; launchConvGemm)
  long wsOff = -1, cntOff = -1;       // split-K workspace / counter offsets (engine-owned)
  int chain = 0;                      // MAXPOOL5: 3 = head of a fused SPPF chain,
                                      // -1 = pooled by the chain head in forward()
};

struct GraphDesc {
  int version = 0;
  std::string task = "detect";
  int nc = 80, imgsz = 0;
  std::vector<BufDesc> bufs;
  std::vector<TenDesc> tens;
  std::vector<OpDesc> ops;
  // derived by validate()
  bool seg = false, obb = false, cls = false;
  int nm = 0, protoTen = -1;
  int probsTen = -1;                  // classify: the SOFTMAX output ([1,1,nc] buffer)
  int detStride = 6;                  // floats per candidate record
  int outK = 6;                       // floats per output record (OBB 7)
  int numAnchors = 0;                 // sum of H*W over the DECODE levels
};

// Parses model.graph (engine/engine.cu:88-141) and checks the invariants the kernels rely
// on (engine/engine.cu:143-191 plus this engine's own: every view %8-aligned).  Returns
// false with a message.
bool parseGraph(const std::string& dir, GraphDesc& g, std::string& err);
bool validateGraph(GraphDesc& g, std::string& err);
// CONV followed by an ADD consuming its output -> CONV with residual (engine/engine.cu:1484).
int fuseAdds(std::vector<OpDesc>& ops);
bool readFile(const std::string& path, std::vector<char>& out, std::string& err);

// ------------------------------------------------------------------ device views
// A tensor view: channel slice [o, o+C) of an NHWC buffer with row stride s (= buffer C).
// Image b, pixel (y, x) of the view starts at p + ((b*H + y)*W + x)*s + o.
struct View {
  f16* p;
  int H, W, s, o, C;
};

// Post-processing parameters, read by kernels from device memory so graphs need no
// re-capture when they change.
struct PostParams {
  float conf;
  float iou;
  int max_det;
  int pad;
};

constexpr int MAX_OUT = 300;          // output records per image (engine/engine.cu:28)
constexpr int NMS_CAP = 2048;         // top-ranked candidates that enter NMS
constexpr int NMS_CLASSES = 1024;     // class ids the NMS kernels bin (ids are < nc <= 1024)
constexpr int NMS_SLACK = 256;        // selected keys beyond NMS_CAP (the boundary bin's ties)
constexpr int NMS_SEL = NMS_CAP + NMS_SLACK;
constexpr int NMS_MASK_WORDS = NMS_CAP * (NMS_CAP / 64);   // bound of one image's mask columns
constexpr int NMS_RANK_SPLIT = 4;     // parts of the selection one rank block compares against
constexpr int NMS_BLOCK_MAX = 512;    // frame graphs: one-block NMS while frames stay this sparse

// Per-image device workspace of the multi-block NMS (one array of Bn of these).
//  sel*   the selected candidates (a superset of the NMS_CAP best keys), in arrival order:
//         key, box, class; selRank[p][i]: (rank << 16 | rank within the class) of key i
//         counted over part p of the selection
//  rIdx   rank -> selected index; cRank / cBox: class-major position -> rank / box
//  cls    present classes in class order: (first class-major position, members, first
//         mask word, -); tile: the class's (first position, members, first mask word) and
//         row chunk << 5 | column chunk
//  mask   per class, column d (members 64d .. 64d+63 as suppressed candidates) holds one
//         word per member i < min(members, 64(d+1)): bit j set iff member i suppresses
//         member 64d + j (i ranked above it); column d starts 32 d (d + 1) words in
//  kept   survivor flags by rank (cleared by the emit kernel for the next frame)
//  Rotated boxes: box = (cx, cy, trace of the covariance or -1 where the far-pair bound does
//  not apply, det) and aux = the covariance (A, B, C, 0).
struct NmsImage {
  unsigned long long selKey[NMS_SEL];
  float4 selBox[NMS_SEL];
  float4 selAux[NMS_SEL];
  int selCls[NMS_SEL];
  unsigned selRank[NMS_RANK_SPLIT][NMS_SEL];
  int rIdx[NMS_CAP];
  int cRank[NMS_CAP];
  float4 cBox[NMS_CAP];
  float4 cAux[NMS_CAP];
  int4 cls[NMS_CLASSES];
  int4 tile[NMS_CAP];
  unsigned kept[NMS_CAP / 32];
  int selN, nClasses, nTiles, pad;
  unsigned long long mask[NMS_MASK_WORDS];
};

// Detection levels handled by one decode launch.
struct DecodeLevel {
  View box, cls, coef;                // coef.p == nullptr for detect
  int H, W, stride, base;             // base = first anchor index of the level
};
struct DecodeArgs {
  DecodeLevel lv[3];                  // OBB: coef is the angle view (channel 0 real)
  int nlev, A, nc, nm, obb;
};

// ------------------------------------------------------------------ GEMM tile configs
struct TileCfg { int BM, BN, WM, WN, BK, NS; };
int numTileConfigs();
const TileCfg& tileConfig(int cfg);

// ------------------------------------------------------------------ launchers
// conv.hip
// One conv as the GEMM launchers take it.
struct ConvJob {
  View x, y;
  const View* res;
  const f16* w;
  const float* bias;
  int k, s, p, act;
};
// Kernel arguments of one implicit-GEMM launch: up to GEMM_GROUP independent convs (problem j
// owns the blocks from blk0), or one conv with split-K (dp, splits, spl, ws, cnt).
constexpr int GEMM_GROUP = 4;
struct GemmProblem {
  View x, y, r;
  const f16* w;
  const float* bias;
  int ksz, cs, cp, act, M, N, Ktot, mtiles, ntiles, xbytes, blk0;
  int m0;   // first output pixel of tile row 0 (0, or where a tail retile starts)
};
struct GemmLaunch {
  GemmProblem p[GEMM_GROUP];
  int n, dp, splits, spl;
  float* ws;
  int* cnt;
};
// Split-K: `splits` > 1 partitions the K stages of every output tile over that many blocks;
// `splits` < -1 does so only for the tiles left over after the last whole wave of the chip
// (tail split, |splits| ways).  `ws` holds |splits| x splitTiles x BM x BN fp32 partials
// (splitWorkspaceBytes) and `cnt` one zeroed counter per split tile (splitTiles), which the
// kernel leaves zeroed again.  Both are sized for M and every smaller batch.
constexpr int MAX_SPLITS = 16;
int splitStages(int Ktot, int BK, int splits);
bool splitOk(int cfg, int Ktot, int splits);
// K iteration mode of a GEMM conv under tile config `cfg` (the kernel is specialised on it):
// KM_ONE  1x1 stride-1 unpadded -- a K stage is BK consecutive channels of one pixel;
// KM_UNI  Cin % BK == 0 (at most 32 taps) -- every stage lies inside one tap, the
//         (channel block, tap) walk is wave-uniform;
// KM_GEN  otherwise -- stages straddle taps, tracked per lane.
constexpr int KM_ONE = 0, KM_UNI = 1, KM_GEN = 2;
int convKMode(int cfg, int k, int s, int p, int Cin);
int numTiles(int cfg, int M, int N);
int tileSlots(int cfg, int km);
int splitTiles(int cfg, int km, int M, int N, int splits);
size_t splitWorkspaceBytes(int cfg, int km, int M, int N, int splits);
// Tail retile: the output tiles of `cfg` that fill whole chip waves (CUs x resident blocks)
// run under `cfg`, and the pixel rows after them under the smaller tile config `tail` in a
// second launch, which spreads that remainder over the chip instead of leaving most CUs idle
// during a part-empty last wave.  `tail` has the same BK, hence the same K walk and the same
// MFMA sequence for every output: the result is bit-identical to `cfg` alone.
bool tailOk(int cfg, int tail, int k, int s, int p, int Cin, int M, int N);
int tailRow(int cfg, int km, int M, int N);   // first pixel of the tail part (M: none)
void launchConvGemm(int cfg, const View& x, const View& y, const View* res, const f16* w,
                    const float* bias, int k, int s, int p, int act, int Bn, int splits,
                    float* ws, int* cnt, hipStream_t st, int tail = -1);
// n independent convs in one launch under tile config `cfg` (all in the same K mode, which
// convGroupOk checks), no split-K; each result equals a launch of that conv alone.
bool convGroupOk(int cfg, const ConvJob* jobs, int n);
void launchConvGemmGroup(int cfg, const ConvJob* jobs, int n, int Bn, hipStream_t st);
// 3x3 stride-1 convs with Cin <= 64 and Cout <= 64 (Cout % 16 == 0): the LDS-halo kernel, an
// autotune candidate selected by the op config CFG_HALO.
constexpr int CFG_HALO = 1000;
bool convHaloOk(const View& x, const View& y, const View* r, int k, int s, int p);
void launchConvHalo(const View& x, const View& y, const View* res, const f16* w, const float* bias, int act,
                    int Bn, hipStream_t st);
// 1x1 stride-1 convs with Cin <= 384 (a multiple of 8) and Cout a multiple of 16: the
// weights-resident streaming kernel, an autotune candidate selected by the op config CFG_1X1.
constexpr int CFG_1X1 = 1001;
bool conv1x1Ok(const View& x, const View& y, const View* r, int k, int s, int p);
void launchConv1x1(const View& x, const View& y, const View* res, const f16* w, const float* bias, int act,
                   int Bn, hipStream_t st);
// The same with two pixel groups of loads in flight per wave and 16-byte stores (identical
// results), selected by the op config CFG_1X1S.
constexpr int CFG_1X1S = 1002;
bool conv1x1StreamOk(const View& x, const View& y, const View* r, int k, int s, int p);
void launchConv1x1Stream(const View& x, const View& y, const View* res, const f16* w, const float* bias,
                         int act, int Bn, hipStream_t st);
// The persistent streaming conv, tile variant v in [0, numTapTiles()): 3x3 stride-1 variants
// (a stage is one 32-channel block of the tile's input halo for all 9 taps) and 1x1 stride-1
// variants, all for Cin % 8 == 0 and Cout % 16 == 0; autotune candidates selected by the op
// configs CFG_TAP + v.
constexpr int CFG_TAP = 1100;
int numTapTiles();
bool convTapOk(int v, const View& x, const View& y, const View* r, int k, int s, int p);
void launchConvTap(int v, const View& x, const View& y, const View* res, const f16* w, const float* bias, int act,
                   int Bn, hipStream_t st);
// The halo-staged 3x3 conv with producer waves (DMA) and consumer waves (MFMA) handing LDS
// ring slots over through counters, tile variant v in [0, numTapWsTiles()): op configs
// CFG_TAPWS + v.  Its waits are bounded spins; convSpinFailures() is the number of waits that
// expired on the current device since the process started (0 unless a launch went wrong, and
// then that launch's outputs are invalid).
constexpr int CFG_TAPWS = 1200;
int numTapWsTiles();
bool convTapWsOk(int v, const View& x, const View& y, const View* r, int k, int s, int p);
void launchConvTapWs(int v, const View& x, const View& y, const View* res, const f16* w, const float* bias, int act,
                     int Bn, hipStream_t st);
int convSpinFailures();
// Op configs that select a kernel other than a GEMM tile (no split-K, no grouped launches).
inline bool specialConvCfg(int cfg) {
  return cfg == CFG_HALO || cfg == CFG_1X1 || cfg == CFG_1X1S || (cfg >= CFG_TAP && cfg < CFG_TAP + numTapTiles()) ||
         (cfg >= CFG_TAPWS && cfg < CFG_TAPWS + numTapWsTiles());
}
// Whether special config `cfg` applies to a conv, and its launch.
bool specialConvOk(int cfg, const View& x, const View& y, const View* r, int k, int s, int p);
void launchSpecialConv(int cfg, const View& x, const View& y, const View* res, const f16* w, const float* bias,
                       int act, int Bn, hipStream_t st);
void launchConvFirst(const View& x, const View& y, const f16* w, const float* bias, int s, int p,
                     int act, int Bn, hipStream_t st);
void launchDwConv(const View& x, const View& y, const View* res, const f16* wt_kkc,
                  const float* bias, int k, int s, int p, int act, int Bn, hipStream_t st);
// n independent depthwise convs in one launch (k_dwconv / k_dwconv3x4 both give the same values)
constexpr int DW_GROUP = 4;
void launchDwConvGroup(const ConvJob* jobs, int n, int Bn, hipStream_t st);
int heuristicTile(int M, int N, int K);
bool tileOk(int cfg, int M, int N, int K);
bool convGemmFits(long inBytes, long wBytes);
// elementwise.hip
void launchAdd(const View& a, const View& b, const View& y, int Bn, hipStream_t st);
void launchMaxPool5(const View& x, const View& y, int Bn, hipStream_t st);
// Three chained MAXPOOL5 (y1 = mp5(x), y2 = mp5(y1), y3 = mp5(y2)) in one launch; the plane
// is held in LDS (sppfPoolLds bytes), so the loader only fuses planes that fit.
size_t sppfPoolLds(int H, int W);
void launchSppfPool(const View& x, const View& y1, const View& y2, const View& y3, int Bn,
                    hipStream_t st);
void launchUpsample2(const View& x, const View& y, int Bn, hipStream_t st);
void launchCopyC(const View& x, const View& y, int Bn, hipStream_t st);
void launchMarker(hipStream_t st);
// n independent channel copies in one launch
constexpr int COPY_GROUP = 8;
void launchCopyCGroup(const View* xs, const View* ys, int n, int Bn, hipStream_t st);
// Kernel arguments of up to COPY_GROUP channel copies run as blocks of a launch: copy i
// moves total[i] 8-channel groups in the blocks from blk0[i] on, blockDim.x groups per
// block (k_copyc, and the copies an attention launch carries after its own blocks).
struct CopyLaunch {
  View x[COPY_GROUP], y[COPY_GROUP];
  int total[COPY_GROUP], blk0[COPY_GROUP];
  int n;
};
// the arguments of n copies at batch Bn in blocks of `threads`; *blocks = blocks they take
CopyLaunch copyLaunch(const View* xs, const View* ys, int n, int Bn, int threads, int* blocks);
void launchPS2(const View& x, const View& y, int Bn, hipStream_t st);
void launchGap(const View& x, const View& y, int Bn, hipStream_t st);
void launchSoftmaxCh(const View& x, const View& y, int Bn, hipStream_t st);
// attention.hip
void attentionInit();
// ncopy channel copies (xs[i] -> ys[i]) independent of the attention may ride in the same
// launch as extra blocks after the attention's own
void launchAttention(const View& qkv, const View& y, int heads, int kd, int hd, int Bn,
                     hipStream_t st, const View* xs = nullptr, const View* ys = nullptr, int ncopy = 0);
// frame.hip
// Source pixel layouts of the preprocess kernels: BGR u8 (3 bytes, the reference's cv::Mat
// layout) or R, G, B, X u8 (4 bytes, how decoders such as PIL hold RGB images in memory).
constexpr int PIXEL_BGR = 0, PIXEL_RGBX = 1;
inline int pixelBytes(int fmt) { return fmt == PIXEL_RGBX ? 4 : 3; }
void launchPreprocessCls(const uint8_t* src, int sh, int sw, f16* dst, int S, int rh, int rw, int top,
                         int left, int fmt, hipStream_t st);
// Letterbox of several frames in one launch (the frame graph's prologue): per-slot source,
// pixel layout, geometry and destination image index, passed by value in chunks of
// LETTERBOX_BATCH.
struct LetterboxSlot {
  const uint8_t* src;
  int sh, sw, top, left, nh, nw, index;
  float scale;
  int fmt;
};
constexpr int LETTERBOX_BATCH = 64;   // 64 x 48 bytes of kernel arguments
// jpeg.hip: the GPU half of the JPEG decode.  One descriptor per component plane (the IDCT
// finds a block's plane by binary search over block0) and one per image (colour kernel).
struct JpegPlane {
  uint32_t block0;       // first block of the plane in the batch's coefficient array
  uint16_t bw, bh;       // block grid
  uint32_t out;          // byte offset of the plane's samples (stride bw * 8)
  uint32_t pad;
  uint16_t q[64];        // dequantisation table, natural order
};
struct JpegFrame {
  uint8_t* dst;          // R, G, B, X frame, W * H * 4 bytes
  int H, W, nc, pad;
  uint32_t plane[3];     // sample offsets of Y, Cb, Cr
  int stride[3], cw[3], ch[3], fh[3], fv[3];
};
void launchJpegIdct(const int16_t* coef, const JpegPlane* planes, int nplanes, int nblocks, uint8_t* samples,
                    hipStream_t st);
void launchJpegColor(const uint8_t* samples, const JpegFrame* frames, int nframes, int maxPixels, hipStream_t st);
struct LetterboxBatch { LetterboxSlot slot[LETTERBOX_BATCH]; };
void launchPreprocessBatch(const LetterboxSlot* slots, int n, f16* dst, int dh, int dw, hipStream_t st);
void launchPreprocess(const uint8_t* src, int sh, int sw, f16* dst, int dh, int dw, float scale,
                      int top, int left, int nh, int nw, hipStream_t st);
// Decode appends each image's survivors as packed (score, anchor) keys to lists[img*A ..]
// and counts[img] (zero on entry; NMS re-arms it).
void launchDecode(const DecodeArgs& a, float* cand, unsigned long long* lists, int* counts,
                  const PostParams* prm, int Bn, hipStream_t st);
void launchNms(const float* cand, unsigned long long* lists, int* counts, int A, int cstride,
               float* out, int* outidx, int* outcnt, int* rawcnt, const PostParams* prm, int Bn,
               hipStream_t st);
// The same NMS (identical results) spread over many CUs: selection, a counting rank, the
// class layout, suppression masks, per-class greedy and the output are six launches over a
// workspace of Bn NmsImage records (zeroed once at allocation; every launch leaves it ready
// for the next frame).
void launchNmsMulti(const float* cand, unsigned long long* lists, int* counts, int A, int cstride,
                    float* out, int* outidx, int* outcnt, int* rawcnt, const PostParams* prm,
                    NmsImage* ws, int Bn, hipStream_t st);
// The rotated fast-NMS (launchNmsObb's results) on the same pipeline: the suppression tiles
// test probiou >= thr, and a candidate is dropped iff any higher-ranked member of its class
// reaches it (an OR per chunk instead of the greedy pass).
void launchNmsObbMulti(const float* cand, unsigned long long* lists, int* counts, int A, float* out,
                       int* outidx, int* outcnt, int* rawcnt, const PostParams* prm, NmsImage* ws,
                       int Bn, hipStream_t st);
// Rotated NMS over 7-float OBB records (cx, cy, w, h, score, cls, theta); output records
// have the same layout.
void launchNmsObb(const float* cand, unsigned long long* lists, int* counts, int A, float* out,
                  int* outidx, int* outcnt, int* rawcnt, const PostParams* prm, int Bn,
                  hipStream_t st);
void launchMasks(const View& proto, const float* cand, int cstride, int A, int nm,
                 const int* outidx, const int* outcnt, const float* outdets, uint8_t* masks,
                 float rx, float ry, int Bn, hipStream_t st);
size_t nmsScratchBytes(int A);

}  // namespace yolo
