/* C ABI of the MI355X (gfx950) YOLOv8 / YOLO11 inference engine.
 *
 * Part 1 re-exports the reference's embedding API with the same names, argument meaning
 * and error behaviour; every declaration cites the reference declaration it replaces
 * (engine/yolo.h in Soju06/yolo11.cu).  The only type change: the stream is a hipStream_t
 * (engine/yolo.h:19 returns cudaStream_t).
 *
 * Part 2 adds extensions the reference has only as CLI modes or not at all: explicit
 * destroy, error-returning create, runtime thresholds, the per-op parity harness (the
 * reference's `dump` mode), the whole-frame graph (its `pipeline` mode), per-op timing
 * (its `profile` mode) and small device/pinned allocation helpers for callers without a
 * GPU allocator of their own.
 *
 * Threading: one stream per handle; a handle is not thread-safe (engine/engine.cu:1656).
 */
#ifndef YOLO_MI355X_H
#define YOLO_MI355X_H

#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ----------------------------------------------------------------------------------
 * Part 1: the reference's embedding API
 * ---------------------------------------------------------------------------------- */

/* engine/yolo.h:7 */
typedef struct { float x1, y1, x2, y2, score; int cls; } YoloDet;
/* engine/yolo.h:8 */
typedef struct { float x, y, w, h, angle, score; int cls; } YoloObbDet;

/* engine/yolo.h:10-11 -- load model dir, fuse, autotune, build and calibrate one hipGraph
 * per B = 1..max_batch.  Like the reference, any load or HIP failure prints a message and
 * calls exit(1); use yolo_create_ex for an error-returning variant. */
void* yolo_create(const char* model_dir, int max_batch);
/* engine/yolo.h:12-16 -- 0 detect, 1 obb, 2 classify, 3 segment. */
int yolo_task(void* h);
/* engine/yolo.h:17-18 -- calibrated latency (ms) of the batch-B graph. */
float yolo_exec_ms(void* h, int B);
/* engine/yolo.h:19 */
hipStream_t yolo_stream(void* h);
/* engine/yolo.h:20-23 -- letterbox a device BGR u8 HWC frame into batch slot `slot`
 * (async on the engine stream; the frame must stay alive until the stream passes it). */
void yolo_preprocess(void* h, const unsigned char* dev_bgr, int height, int width, int slot);
/* engine/yolo.h:24-25 -- launch the batch-B graph and wait. */
void yolo_run(void* h, int B);
/* engine/yolo.h:26-28 */
void yolo_run_async(void* h, int B);
void yolo_sync(void* h);
/* engine/yolo.h:29-30 -- detections of a slot in original-image coordinates; returns
 * min(count, cap). */
int yolo_get(void* h, int slot, YoloDet* out, int cap);
/* engine/yolo.h:31-35 -- classify models: resize the shortest edge to S with the antialiased
 * bilinear filter, centre-crop S x S, /255, into batch slot `slot` (async on the engine
 * stream); yolo_get_cls writes the top-k class ids and probabilities of a slot after a run
 * and returns min(k, nc), or 0 on a non-classify handle (engine/engine.cu:1758-1773). */
void yolo_preprocess_cls(void* h, const unsigned char* dev_bgr, int height, int width, int slot);
int yolo_get_cls(void* h, int slot, int* ids, float* probs, int k);
/* engine/yolo.h:36-38 */
void yolo_slot_geom(void* h, int slot, float* scale, int* top, int* left);
/* engine/yolo.h:39-41 -- rotated boxes of an OBB handle in original-image coordinates
 * (centre x, y and w, h divided by the letterbox scale, angle in radians unchanged, no
 * clipping); returns the count written.  Returns 0 on detect/segment handles, and
 * yolo_get returns 0 on OBB handles (the reference reads the wrong record stride there). */
int yolo_get_obb(void* h, int slot, YoloObbDet* out, int cap);
/* engine/yolo.h:42-43 */
void yolo_mask_dim(void* h, int* ph, int* pw);
/* engine/yolo.h:44-49 -- binary mask of detection `det` of `slot` (ph*pw bytes); 0 or -1. */
int yolo_get_mask(void* h, int slot, int det, unsigned char* out);

/* ----------------------------------------------------------------------------------
 * Part 2: extensions (no counterpart in engine/yolo.h unless cited)
 * ---------------------------------------------------------------------------------- */

#define YOLO_NOFUSE 1      /* keep CONV+ADD pairs separate (the reference's NOFUSE / dump)  */
#define YOLO_NOTUNE 2      /* skip the startup tile autotuner (the reference's NOTUNE)       */
#define YOLO_NOGRAPH 4     /* do not capture per-B graphs at create (yolo_run then streams)  */
#define YOLO_BRANCHES 8    /* eager (non-graph) forward runs independent branches on 3 side
                              streams                                                      */
#define YOLO_DAGGRAPH 16   /* graphs are a dependency DAG of per-op kernel nodes (independent
                              branches may run concurrently) instead of one single-stream
                              capture; slower for batch 1 on ROCm 7.2                      */
#define YOLO_NOGROUP 32    /* one op per launch: no grouped launches of independent convs /
                              copies (results are identical either way)                    */
#define YOLO_NMS_BLOCK 64  /* NMS (detect, segment, rotated) in one block per image (one
                              launch) instead of the multi-block pipeline (six launches
                              spread over the GPU); identical results                      */

/* Batch staging and fetch for servers (one call per batch instead of one per slot; the
 * reference server stages and reads per slot, server/serve.cpp:264-302):
 * yolo_stage_frames copies B raw u8 HWC frames of pixel layout `format` from host memory
 * into the handle's own device staging buffers and letterboxes them (classify handles: the
 * resize + centre crop) into slots 0..B-1, asynchronously on the engine stream; pinned host
 * memory (yolo_host_alloc) makes the copies asynchronous, and it must stay valid until the
 * stream passes them (e.g. the next yolo_sync).  Both layouts give identical results; RGBX
 * is how image decoders hold RGB in memory, so a server can stage their buffer unconverted.
 * Returns 0, or -1 on bad arguments.
 * yolo_get_batch / yolo_get_obb_batch write slot s's detections (as yolo_get /
 * yolo_get_obb) to out[s * cap ...] and their number to counts[s]; return the total. */
#define YOLO_PIXEL_BGR 0   /* B, G, R bytes per pixel (the reference's cv::Mat layout)      */
#define YOLO_PIXEL_RGBX 1  /* R, G, B, X bytes per pixel (X ignored)                        */
int yolo_stage_frames(void* h, int B, const unsigned char* const* host, const int* heights,
                      const int* widths, int format, int first_slot);

/* JPEG frames decoded by the engine, as the reference server does with nvJPEG (CPU Huffman
 * across decoder threads, the rest on the GPU; server/serve.cpp:71-131): entropy decoding on
 * the library's decoder threads (one stream per thread, YOLO_DECODE_THREADS or the process's
 * CPUs up to 16), then dequantisation + IDCT, chroma upsampling and YCbCr -> RGB as GPU
 * kernels, then the letterbox (classify: resize + crop) into slots first_slot..first_slot+B-1.
 * The pixels equal PIL's / libjpeg-turbo's decode of the same bytes exactly (integer "islow"
 * IDCT, "fancy" upsampling, 16-bit fixed-point colour).  Baseline / extended-sequential
 * Huffman 8-bit streams with one scan, grayscale or YCbCr, chroma subsampled by at most 2
 * each way; status[i] says whether stream i was staged, is outside that set (decode it
 * another way and stage it with yolo_stage_frames), or is corrupt / truncated.  Returns when
 * the entropy decoding is done (copies and kernels are queued on the engine stream): the
 * number of streams not staged, or -1 on bad arguments.  heights / widths (optional) receive
 * each staged stream's size.
 * yolo_jpeg_probe reads only the headers: 1 = yolo_stage_jpeg decodes it (size in *height /
 * *width), 0 = a JPEG outside that set, -1 = not a JPEG or a malformed header.
 * yolo_jpeg_coefficients (host code only, no GPU) entropy-decodes a stream into its quantised
 * coefficients, int16 in natural order, component plane after plane, block-row-major; returns
 * the count (out == NULL: the count needed), -1 if unsupported / cap too small, -2 if corrupt. */
#define YOLO_JPEG_STAGED 0
#define YOLO_JPEG_UNSUPPORTED 1
#define YOLO_JPEG_INVALID 2
int yolo_stage_jpeg(void* h, int B, const unsigned char* const* data, const size_t* sizes, int first_slot,
                    int* heights, int* widths, int* status);
/* yolo_stage_jpeg in two steps, so a pipelined caller can decode the next batch while the
 * current one runs and still read the current one's results (their letterbox geometry is
 * the slots' until the next letterbox): yolo_decode_jpeg decodes into the slots' staging
 * frames only (same arguments and return value); yolo_letterbox_decoded letterboxes the
 * frames it left in slots first_slot..first_slot+B-1 (skipping slots whose decode failed or
 * that were restaged since) and returns how many, or -1 on bad arguments. */
int yolo_decode_jpeg(void* h, int B, const unsigned char* const* data, const size_t* sizes, int first_slot,
                     int* heights, int* widths, int* status);
int yolo_letterbox_decoded(void* h, int B, int first_slot);
/* Decoding at arrival, for servers: yolo_jpeg_submit copies a stream, reads its headers and
 * starts its entropy decoding on the decoder threads at once (into pinned memory), returning a
 * ticket, or NULL if the stream is not one yolo_stage_jpeg decodes (decode it another way).
 * yolo_decode_tickets is yolo_decode_jpeg for B tickets: it waits for each one's entropy
 * decoding (usually long done), copies the coefficients and runs the GPU half; it consumes
 * every ticket passed (NULL entries are reported corrupt).  yolo_jpeg_release frees a ticket
 * that will not be decoded (after its entropy decoding ends). */
void* yolo_jpeg_submit(const unsigned char* data, size_t size);
int yolo_decode_tickets(void* h, int B, void* const* tickets, int first_slot, int* heights, int* widths,
                        int* status);
void yolo_jpeg_release(void* ticket);
int yolo_jpeg_probe(const unsigned char* data, size_t size, int* height, int* width);
/* Threads (the calling one included) the JPEG entropy decoding runs on; -1 if they cannot be
 * started. */
int yolo_decoder_threads(void);
/* The largest frame, in pixels (height x width), the engine decodes: larger JPEG streams are
 * reported outside the set (yolo_jpeg_probe 0, yolo_jpeg_submit NULL, status
 * YOLO_JPEG_UNSUPPORTED), since a header of a few bytes can declare a 65535 x 65535 frame
 * whose coefficients the decoder would have to hold.  n > 0 sets it (process-wide); returns
 * the value in force.  The default is PIL's Image.MAX_IMAGE_PIXELS, 89,478,485.  Streams of a
 * batch that would push its coefficient or sample buffers past 2^31 blocks or 2^32 bytes are
 * likewise reported YOLO_JPEG_UNSUPPORTED, and the rest of the batch is staged. */
long long yolo_jpeg_max_pixels(long long n);
long long yolo_jpeg_coefficients(const unsigned char* data, size_t size, short* out, size_t cap);
int yolo_get_batch(void* h, int B, YoloDet* out, int cap, int* counts);
int yolo_get_obb_batch(void* h, int B, YoloObbDet* out, int cap, int* counts);

/* Masks of detections first..first+n-1 of a slot (n * ph * pw bytes, one copy); 0, or -1
 * on bad arguments.  yolo_get_mask (engine/yolo.h:44-49) for a range. */
int yolo_get_masks(void* h, int slot, int first, int n, unsigned char* out);

/* The server's batch worker (server/serve.cpp:165-191 batcher, :264-302 worker loop), native:
 * requests are submitted from any thread; one worker thread collects a model's queue when it
 * is full or its oldest request would otherwise miss target_ms (slack = target - age -
 * yolo_exec_ms(max batch) - staging estimate - 1 ms), runs the GPU half of its JPEG decodes
 * beside the previous batch, reads the previous batch's results, stages (letterboxes) and
 * launches the batch.  Engines belong to the batcher's thread while it runs: make no other
 * call on them.  Batches never mix models.
 * yolo_batcher_submit_jpeg: 0 queued (the engine decodes the stream; its entropy decoding
 * starts now), 1 not a stream the engine decodes (decode it another way and submit the
 * pixels), -1 stopped / bad arguments.  yolo_batcher_submit_frame: R, G, B, X pixels in host
 * memory (pinned for asynchronous copies) that must stay valid until the request's result is
 * collected (it is returned in `host`); 0 or -1.
 * yolo_batcher_wait: collects up to cap finished requests (waits up to timeout_ms, < 0 for
 * ever); returns the count, 0 on timeout, -1 once stopped and every request answered.  Each
 * result stays valid until yolo_batcher_release.  rows: n records of `stride` floats --
 * detect / segment (x1, y1, x2, y2, score, cls) in original-image coordinates, OBB (cx, cy,
 * w, h, angle, score, cls), classify the top-5 (cls, prob); segment also the RLE of each
 * mask at proto resolution (alternating 0/1 runs starting with a 0-run, row-major;
 * server/serve.cpp:193-203): rle_len[j] runs of mask j, concatenated in rle, and the
 * letterbox geometry.  queue_ms: arrival to launch; infer_ms: launch to results.
 * yolo_batcher_stop: no new requests; queued ones are answered with YOLO_BATCH_STOPPED. */
#define YOLO_BATCH_OK 0
#define YOLO_BATCH_DECODE_FAILED 1  /* corrupt stream, or past what one batch decode holds */
#define YOLO_BATCH_STOPPED 2
#define YOLO_BATCH_FAILED 3         /* the batch could not be staged or its results built (host memory) */
typedef struct {
  long long tag;
  int status, model, task, batch;
  float queue_ms, infer_ms;
  int n, stride;
  const float* rows;
  const unsigned* rle;
  const int* rle_len;
  int mask_h, mask_w;
  float lb_scale;
  int lb_top, lb_left;
  const unsigned char* host;   /* the frame passed to yolo_batcher_submit_frame, or NULL */
  void* owner;
} YoloBatchResult;
void* yolo_batcher_create(void* const* engines, const int* max_batch, int n, double target_ms);
int yolo_batcher_submit_jpeg(void* b, int model, const unsigned char* data, size_t size, long long tag);
int yolo_batcher_submit_frame(void* b, int model, const unsigned char* rgbx, int height, int width,
                              long long tag);
int yolo_batcher_wait(void* b, YoloBatchResult* out, int cap, int timeout_ms);
void yolo_batcher_release(const YoloBatchResult* r, int n);
double yolo_batcher_stage_ms(void* b);
void yolo_batcher_stop(void* b);
void yolo_batcher_destroy(void* b);

/* Error-returning create: NULL on failure with a message in err (if non-NULL). */
void* yolo_create_ex(const char* model_dir, int max_batch, int flags, char* err, int errlen);
/* The reference has no destroy (the handle lives until exit); this frees everything. */
void yolo_destroy(void* h);
/* Parse and validate a model dir on the host only (no GPU needed).  Returns the op count
 * after loading, or -1 with a message in err.  Same grammar and invariants as
 * loadGraph (engine/engine.cu:88-191). */
int yolo_graph_check(const char* model_dir, char* err, int errlen);
/* Runtime post-processing parameters.  The reference hard-codes conf 0.25, IoU 0.45 and
 * 300 outputs (engine/engine.cu:1411,1466,28); these live in device memory so captured
 * graphs pick them up without re-capture.  max_det <= 300.  Returns 0 or -1. */
int yolo_set_thresholds(void* h, float conf, float iou, int max_det);
/* Candidates that passed conf before NMS for a slot in the last run (the reference's
 * h_rawcnt truncation tripwire, engine/engine.cu:1538-1546). */
int yolo_raw_count(void* h, int slot);

/* Per-op parity harness -- the reference's `dump` mode (engine/engine.cu:1843-1888). */
int yolo_num_ops(void* h);
/* info[0..8] = kind, a, b, out, k, s, g, Cin, Cout.  Kinds: 0 CONV, 1 ADD, 2 MAXPOOL5,
 * 3 UPSAMPLE2, 4 COPYC, 5 ATTN, 6 DECODE, 7 GAP, 8 SOFTMAX, 9 DECODEOBB, 10 PS2,
 * 11 DECODESEG, 12 MASKS (the reference's OpKind order, engine/engine.cu:33-34). */
int yolo_op_info(void* h, int k, int* info);
int yolo_num_tensors(void* h);
/* hwc[0..2] = H, W, C of tensor t. */
int yolo_tensor_shape(void* h, int t, int* hwc);
/* Copy tensor t of the first B images to/from contiguous host fp16 [B][H][W][C]. */
int yolo_read_tensor(void* h, int t, int B, void* host_f16);
int yolo_write_tensor(void* h, int t, int B, const void* host_f16);
/* The same for images first .. first+n-1 only. */
int yolo_read_tensor_slots(void* h, int t, int first, int n, void* host_f16);
int yolo_write_tensor_slots(void* h, int t, int first, int n, const void* host_f16);
/* Run op k alone for B images on the engine stream and wait.  Returns 0 or -1. */
int yolo_run_op(void* h, int k, int B);
/* Run NMS (+ masks) and the result copies for B images after the DECODE ops ran. */
int yolo_run_post(void* h, int B);
/* Tile configuration the dispatcher uses for a CONV op (autotuned or heuristic), and an
 * override (cfg < 0 restores the heuristic).  Returns -1 for non-GEMM ops.  cfg 1000 selects
 * the LDS-halo kernel for 3x3 stride-1 convs with Cin <= 64 and Cout <= 64 (Cout a multiple
 * of 16), cfg 1001 the weights-resident kernel for 1x1 stride-1 convs with Cin <= 384 (a
 * multiple of 8) and Cout a multiple of 16, cfgs 1100 .. 1112 the tile variants of the
 * persistent streaming conv: 1100 .. 1107 for 3x3 stride-1 convs (one LDS stage = a 32-channel
 * block of the output tile's input halo for all 9 taps), 1108 .. 1112 for 1x1 stride-1 convs,
 * both with Cin a multiple of 8 and Cout a multiple of 16; set_op_config refuses them for
 * other convs. */
int yolo_op_config(void* h, int k);
int yolo_set_op_config(void* h, int k, int cfg);   /* also resets the op's split-K to 1 */
/* Split-K factor of a GEMM CONV op (autotuned at create, 1 = none) and an override: the K
 * stages are divided over `splits` blocks per output tile whose fp32 partials are summed in
 * split order (deterministic).  A negative value -S is a tail split: the output tiles that
 * fill whole waves of the chip run unsplit and only the remaining tiles (the part-empty last
 * wave) are split S ways.  The override is refused (-1) once graphs are captured
 * (YOLO_NOGRAPH handles only), for non-GEMM ops and for splits that leave a block empty. */
int yolo_op_split(void* h, int k);
int yolo_set_op_split(void* h, int k, int splits);
/* Tail retile of GEMM conv k (no counterpart in engine/yolo.h; a tuning and parity hook like
 * the split override): the output tiles of the op's tile config that fill whole waves of the
 * chip run under that config, and the pixel rows after them under the smaller tile config
 * `tail` (same K per stage) in a second launch, so the part-empty last wave is spread over
 * the chip.  Results are bit-identical to the op's config alone.  -1 clears it; refused (-1)
 * for non-GEMM ops, split ops, and tails that do not apply.  yolo_op_tail returns the tail
 * config, -1 for none, -2 for a bad op.  The autotuner sets it where it is faster; graphs
 * captured before a change keep the launches they were captured with. */
int yolo_op_tail(void* h, int k);
int yolo_set_op_tail(void* h, int k, int tail);
/* Number of GEMM tile configurations compiled in, and the shape of one:
 * out[0..5] = BM (pixels), BN (channels), waves along M, waves along N, BK (K per stage),
 * LDS ring stages. */
int yolo_num_tile_configs(void);
int yolo_tile_config(int cfg, int* out);

/* Whole-frame graph -- the reference's `pipeline` mode (engine/engine.cu:1974-2032):
 * one graph holding [H2D of each raw frame] + letterbox of each slot + network + decode +
 * NMS + result copies.  host_bgr may be NULL (frames already in device memory) or an
 * array of B pinned host pointers.  Replaces any previous frame graph.  Two variants are
 * captured (unless YOLO_NMS_BLOCK): the launch takes the one-block NMS while the previous
 * frame's results showed at most 512 candidates in every slot, else the multi-block NMS;
 * the detections are identical either way. */
int yolo_frame_graph(void* h, int B, const unsigned char* const* dev_bgr,
                     const unsigned char* const* host_bgr, const int* heights, const int* widths);
int yolo_frame_run(void* h);       /* launch + wait */
int yolo_frame_launch(void* h);    /* launch only    */

/* Timing on the engine stream with hipEvents (the reference's `bench`/`profile` modes,
 * engine/engine.cu:2033-2090). */
/* Average ms of `iters` launches of the batch-B graph (which = 0) or frame graph (1). */
float yolo_time_graph(void* h, int which, int B, int iters);
/* Per-op average ms over `iters` stream-ordered passes (ms[k] for every op k).  An op executed
 * inside a preceding op's launch (the second and third MAXPOOL5 of a fused SPPF chain)
 * reports only its event overhead. */
int yolo_profile_ops(void* h, int B, int iters, float* ms);
/* Kernel time per launch unit: each unit (one op, or a group of independent ops launched
 * together) runs `reps` times back to back between two events, so the per-launch gaps of a
 * stream-ordered pass are not counted; ms[k] is the average per run over `iters` passes,
 * reported on the unit's first op (0 on the other members, on decode ops and on pooled ops
 * of a fused SPPF chain).  Activations are left in an unspecified state. */
int yolo_profile_units(void* h, int B, int iters, int reps, float* ms);
/* The launch unit op k runs in (ops of one unit share a launch; units are numbered in launch
 * order), -1 for ops no unit launches (decode ops, pooled ops of a fused SPPF chain), -2 for
 * a bad op index. */
int yolo_op_unit(void* h, int k);
/* Launch units of the handle, and one unit u at batch B on the engine stream, asynchronously
 * (0; -1 on bad arguments; units of decode ops launch nothing).  yolo_marker queues an empty
 * one-wave kernel (k_marker) on the engine stream: a profiler sees it as a separator, so a
 * trace of marker, unit, marker, unit, ... attributes every dispatch to its unit. */
int yolo_num_units(void* h);
int yolo_run_unit(void* h, int u, int B);
int yolo_marker(void* h);
/* Number of bounded waits that expired in kernels whose waves hand work to each other through
 * LDS counters (the wave-specialised conv, op configs 1200+) on the handle's device since the
 * process started: 0 unless such a launch went wrong, and then that launch's outputs are
 * invalid.  No counterpart in the reference; -1 on a device error. */
int yolo_spin_failures(void* h);
/* Average ms of the frame's pre/post stages over `iters` stream-ordered passes of the frame
 * set by yolo_frame_graph (frames in device memory, no H2D): ms[0] letterbox of all slots,
 * ms[1] decode (all levels, one launch), ms[2] NMS, ms[3] mask assembly (0 without a proto).
 * -1 on classify handles or before yolo_frame_graph. */
int yolo_profile_stages(void* h, int iters, float* ms);

/* Allocation helpers (device / pinned host) and copies on the engine stream. */
void* yolo_dev_alloc(size_t bytes);
void yolo_dev_free(void* p);
void* yolo_host_alloc(size_t bytes);
void yolo_host_free(void* p);
int yolo_copy_h2d(void* h, void* dst, const void* src, size_t bytes);
int yolo_copy_d2h(void* h, void* dst, const void* src, size_t bytes);

/* Decode + NMS of caller-provided detect heads that allocates nothing.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid hipMalloc) and have their own network output.  It is
 * the handle-free form of a detect handle's DECODE ops + yolo_run_post, with the same kernels
 * and results: box views hold 64 DFL bins, cls views ceil8(nc) logits (pad channels
 * ignored), NHWC fp16 with a row stride and first channel in halves (multiples of 8,
 * 16-byte aligned base).  Outputs (device memory): dets [B][300][6] letterbox-space
 * x1 y1 x2 y2 score cls in NMS order, counts [B] kept, raw_counts [B] (may be NULL)
 * candidates that passed conf.  Asynchronous on `stream`.  Scratch is one fixed device
 * array per GPU (YOLO_STATIC_MAX_ANCHOR_SLOTS anchors over the batch, at most
 * YOLO_STATIC_MAX_BATCH images; about 5.3 MB): larger inputs are refused with -1, and calls
 * that overlap on one GPU race.  Returns 0 or -1 (message on stderr). */
#define YOLO_STATIC_MAX_BATCH 64
#define YOLO_STATIC_MAX_ANCHOR_SLOTS 163840
typedef struct {
  const void* box;                 /* [B][H][W][box_stride] fp16, bins at box_off..+64     */
  const void* cls;                 /* [B][H][W][cls_stride] fp16, logits at cls_off..+nc   */
  int H, W, stride;                /* grid size and stride (pixels per cell) of the level  */
  int box_stride, box_off, cls_stride, cls_off;
} YoloHeadLevel;
int yolo_detect_static(const YoloHeadLevel* levels, int nlev, int B, int nc, float conf, float iou,
                       int max_det, float* dets, int* counts, int* raw_counts, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* YOLO_MI355X_H */
