// Model-dir parser and validator (host only, no HIP calls).
//
// Grammar follows the reference loader (engine/engine.cu:88-141, written by
// export/export.py:709-717):
//   YOLO11GRAPH <ver>
//   TASK <task> <nc> <imgsz>                      (ver >= 2)
//   <nbufs> <ntens> <nops>
//   B <H> <W> <C>          x nbufs
//   T <buf> <coff> <C>     x ntens
//   <TAG> <ints...>        x nops   (CONV 11, ADD 3, ATTN 5, DECODE 3, DECODESEG 4, ...)
// Validation restates the reference's load-time invariants (engine/engine.cu:143-191) and
// adds the ones this engine's kernels need (16-byte aligned channel views, shapes that
// agree with each op's arithmetic), reporting errors instead of exiting.
#include "engine.hpp"

#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>

namespace yolo {

bool readFile(const std::string& path, std::vector<char>& out, std::string& err) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) { err = "cannot open " + path; return false; }
  fseek(f, 0, SEEK_END);
  long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  out.resize(n > 0 ? n : 0);
  size_t rd = n > 0 ? fread(out.data(), 1, n, f) : 0;
  fclose(f);
  if ((long)rd != n) { err = "short read " + path; return false; }
  return true;
}

static bool opArity(const std::string& tag, int& kind, int& n) {
  static const struct { const char* t; int kind, n; } table[] = {
      {"CONV", CONV, 11},         {"ADD", ADD, 3},     {"MAXPOOL5", MAXPOOL5, 2},
      {"UPSAMPLE2", UPSAMPLE2, 2}, {"COPYC", COPYC, 2}, {"ATTN", ATTN, 5},
      {"DECODE", DECODE, 3},      {"GAP", GAP, 2},     {"SOFTMAX", SOFTMAX, 2},
      {"DECODEOBB", DECODEOBB, 4}, {"PS2", PS2, 2},    {"DECODESEG", DECODESEG, 4},
      {"MASKS", MASKS, 1}};
  for (const auto& e : table)
    if (tag == e.t) { kind = e.kind; n = e.n; return true; }
  return false;
}

bool parseGraph(const std::string& dir, GraphDesc& g, std::string& err) {
  std::ifstream f(dir + "/model.graph");
  if (!f) { err = "no model.graph in " + dir; return false; }
  std::string magic, tag;
  if (!(f >> magic >> g.version)) { err = "bad graph header"; return false; }
  if (g.version >= 2) {
    if (!(f >> tag >> g.task >> g.nc >> g.imgsz) || tag != "TASK") {
      err = "bad TASK header";
      return false;
    }
  }
  int nb, nt, no;
  if (!(f >> nb >> nt >> no) || nb <= 0 || nt <= 0 || no < 0) { err = "bad counts line"; return false; }
  g.bufs.resize(nb);
  g.tens.resize(nt);
  for (int i = 0; i < nb; i++)
    if (!(f >> tag >> g.bufs[i].H >> g.bufs[i].W >> g.bufs[i].C) || tag != "B") {
      err = "bad buffer line " + std::to_string(i);
      return false;
    }
  for (int i = 0; i < nt; i++)
    if (!(f >> tag >> g.tens[i].buf >> g.tens[i].coff >> g.tens[i].C) || tag != "T") {
      err = "bad tensor line " + std::to_string(i);
      return false;
    }
  for (int i = 0; i < no; i++) {
    int kind, n;
    if (!(f >> tag)) { err = "missing op " + std::to_string(i); return false; }
    if (!opArity(tag, kind, n)) { err = "bad op " + tag; return false; }
    long v[11];
    for (int j = 0; j < n; j++)
      if (!(f >> v[j])) { err = "short op line " + std::to_string(i) + " (" + tag + ")"; return false; }
    OpDesc op;
    op.kind = kind;
    switch (kind) {
      case CONV:
        op.a = v[0]; op.out = v[1]; op.k = v[2]; op.s = v[3]; op.p = v[4]; op.g = v[5];
        op.act = v[6]; op.Cin = v[7]; op.Cout = v[8]; op.woff = v[9]; op.boff = v[10];
        break;
      case ADD: op.a = v[0]; op.b = v[1]; op.out = v[2]; break;
      case ATTN: op.a = v[0]; op.out = v[1]; op.heads = v[2]; op.kd = v[3]; op.hd = v[4]; break;
      case DECODE: op.a = v[0]; op.b = v[1]; op.stride = v[2]; break;
      case DECODEOBB:
      case DECODESEG: op.a = v[0]; op.b = v[1]; op.out = v[2]; op.stride = v[3]; break;
      case MASKS: op.a = v[0]; break;
      default: op.a = v[0]; op.out = v[1]; break;
    }
    g.ops.push_back(op);
  }
  return true;
}

namespace {
struct Shape { int H, W, C; };
}

bool validateGraph(GraphDesc& g, std::string& err) {
  const int nb = g.bufs.size(), nt = g.tens.size();
  auto bad = [&](const std::string& m) { err = m; return false; };
  for (int i = 0; i < nb; i++) {
    const auto& b = g.bufs[i];
    if (b.H <= 0 || b.W <= 0 || b.C <= 0) return bad("buffer " + std::to_string(i) + " has a non-positive dim");
  }
  for (int i = 0; i < nt; i++) {
    const auto& t = g.tens[i];
    if (t.buf < 0 || t.buf >= nb) return bad("tensor " + std::to_string(i) + " names a missing buffer");
    if (t.coff < 0 || t.C <= 0 || t.coff + t.C > g.bufs[t.buf].C)
      return bad("tensor " + std::to_string(i) + " exceeds its buffer");
  }
  auto tenOk = [&](int t) { return t >= 0 && t < nt; };
  auto shp = [&](int t) { const auto& T = g.tens[t]; const auto& B = g.bufs[T.buf]; return Shape{B.H, B.W, T.C}; };
  // vec8 views: channel offset, width and row stride all multiples of 8 halves (16 bytes)
  auto al8 = [&](int t) {
    const auto& T = g.tens[t];
    return T.coff % 8 == 0 && T.C % 8 == 0 && g.bufs[T.buf].C % 8 == 0;
  };
  // tensor 0 is the network input; the letterbox entry points require it to be a
  // standalone 3-channel buffer and check that when called (single-op test graphs feed
  // other shapes through yolo_write_tensor)
  const Shape in = shp(0);
  if (g.imgsz && (in.H != g.imgsz || in.W != g.imgsz)) return bad("imgsz header mismatch");
  if (g.tens[0].coff != 0) return bad("input tensor must start at channel 0 of its buffer");
  if (g.task != "detect" && g.task != "segment" && g.task != "obb" && g.task != "classify")
    return bad("unknown task " + g.task);
  g.seg = g.task == "segment";
  g.obb = g.task == "obb";
  g.cls = g.task == "classify";

  int nlev = 0;
  g.numAnchors = 0;
  for (size_t i = 0; i < g.ops.size(); i++) {
    const OpDesc& op = g.ops[i];
    const std::string at = "op " + std::to_string(i) + ": ";
    switch (op.kind) {
      case CONV: {
        if (!tenOk(op.a) || !tenOk(op.out)) return bad(at + "tensor id out of range");
        Shape x = shp(op.a), y = shp(op.out);
        if (op.k <= 0 || op.s <= 0 || op.p < 0) return bad(at + "bad k/s/p");
        int Ho = (x.H + 2 * op.p - op.k) / op.s + 1, Wo = (x.W + 2 * op.p - op.k) / op.s + 1;
        if (x.C != op.Cin || y.C != op.Cout) return bad(at + "CONV channel counts disagree with its views");
        if (y.H != Ho || y.W != Wo) return bad(at + "CONV output size disagrees with k/s/p");
        if (op.woff < 0 || op.boff < 0) return bad(at + "negative weight offset");
        if (op.g == 1) {
          if (op.Cin == 3) {
            if (op.Cout % 8 || !al8(op.out)) return bad(at + "first conv needs an 8-aligned output view");
            if (op.k != 3 || op.Cout > 256) return bad(at + "first conv (Cin 3) must be 3x3 with Cout <= 256");
            if (g.bufs[g.tens[op.a].buf].C != 3) return bad(at + "first conv input must be a 3-channel buffer");
          } else {
            if (!al8(op.a) || !al8(op.out)) return bad(at + "GEMM conv needs 8-aligned views (Cin, Cout, offsets, strides)");
            if (op.woff % 8) return bad(at + "GEMM conv weight offset must be 8-aligned");
          }
        } else {
          if (op.g != op.Cin || op.Cin != op.Cout) return bad(at + "only depthwise grouped convs are supported");
          if (!al8(op.a) || !al8(op.out)) return bad(at + "depthwise conv needs 8-aligned views");
          if (op.woff % 8) return bad(at + "depthwise conv weight offset must be 8-aligned");
        }
        break;
      }
      case ADD: {
        if (!tenOk(op.a) || !tenOk(op.b) || !tenOk(op.out)) return bad(at + "tensor id out of range");
        Shape a = shp(op.a), b = shp(op.b), y = shp(op.out);
        if (a.H != b.H || a.W != b.W || a.C != b.C || a.H != y.H || a.W != y.W || a.C != y.C)
          return bad(at + "ADD shapes differ");
        if (!al8(op.a) || !al8(op.b) || !al8(op.out)) return bad(at + "ADD needs 8-aligned views");
        break;
      }
      case MAXPOOL5:
      case COPYC:
      case UPSAMPLE2:
      case PS2: {
        if (!tenOk(op.a) || !tenOk(op.out)) return bad(at + "tensor id out of range");
        Shape x = shp(op.a), y = shp(op.out);
        if (!al8(op.a) || !al8(op.out)) return bad(at + "needs 8-aligned views");
        if (op.kind == MAXPOOL5 || op.kind == COPYC) {
          if (x.H != y.H || x.W != y.W || x.C != y.C) return bad(at + "shapes differ");
        } else if (op.kind == UPSAMPLE2) {
          if (y.H != 2 * x.H || y.W != 2 * x.W || y.C != x.C) return bad(at + "UPSAMPLE2 shape");
        } else {
          if (y.H != 2 * x.H || y.W != 2 * x.W || x.C != 4 * y.C) return bad(at + "PS2 shape");
        }
        break;
      }
      case ATTN: {
        if (!tenOk(op.a) || !tenOk(op.out)) return bad(at + "tensor id out of range");
        Shape q = shp(op.a), y = shp(op.out);
        if (op.heads <= 0 || op.kd != 32 || op.hd <= 0 || op.hd % 16 || op.hd > 128)
          return bad(at + "ATTN needs kd == 32 and hd a multiple of 16 up to 128");
        if (q.C != op.heads * (2 * op.kd + op.hd) || y.C != op.heads * op.hd || q.H != y.H || q.W != y.W)
          return bad(at + "ATTN channel layout");
        if (!al8(op.a) || !al8(op.out)) return bad(at + "ATTN needs 8-aligned views");
        break;
      }
      case GAP: {
        if (!tenOk(op.a) || !tenOk(op.out)) return bad(at + "tensor id out of range");
        Shape x = shp(op.a), y = shp(op.out);
        if (y.H != 1 || y.W != 1 || y.C != x.C) return bad(at + "GAP output must be [1,1,C] of its input's C");
        if (!al8(op.a) || !al8(op.out)) return bad(at + "GAP needs 8-aligned views");
        break;
      }
      case SOFTMAX: {
        if (!tenOk(op.a) || !tenOk(op.out)) return bad(at + "tensor id out of range");
        Shape x = shp(op.a), y = shp(op.out);
        if (x.H != 1 || x.W != 1 || y.H != 1 || y.W != 1 || x.C != y.C)
          return bad(at + "SOFTMAX works on [1,1,C] views of equal C");
        if (!g.cls) return bad(at + "SOFTMAX needs task=classify");
        g.probsTen = op.out;
        break;
      }
      case DECODE:
      case DECODESEG:
      case DECODEOBB: {
        if (g.cls) return bad(at + "classify graphs have no DECODE ops");
        if (!tenOk(op.a) || !tenOk(op.b)) return bad(at + "tensor id out of range");
        Shape bx = shp(op.a), c = shp(op.b);
        if (bx.C != 64) return bad(at + "DECODE box view must have 64 channels (4 x reg_max 16)");
        if (c.C % 8 || c.C < g.nc) {
          char m[160];
          snprintf(m, sizeof m, "DECODE needs an 8-aligned cls view covering nc (nc=%d, C=%d)", g.nc, c.C);
          return bad(at + m);
        }
        if (bx.H != c.H || bx.W != c.W) return bad(at + "DECODE box/cls sizes differ");
        if (!al8(op.a) || !al8(op.b)) return bad(at + "DECODE needs 8-aligned views");
        if (op.kind == DECODESEG) {
          if (!g.seg) return bad(at + "DECODESEG needs task=segment");
          if (!tenOk(op.out)) return bad(at + "tensor id out of range");
          Shape m = shp(op.out);
          if (m.H != bx.H || m.W != bx.W || !al8(op.out)) return bad(at + "DECODESEG coef view");
        } else if (op.kind == DECODEOBB) {
          // engine/engine.cu:161-167: the angle view is %8-padded, channel 0 real
          if (!g.obb) return bad(at + "DECODEOBB needs task=obb");
          if (!tenOk(op.out)) return bad(at + "tensor id out of range");
          Shape an = shp(op.out);
          if (an.H != bx.H || an.W != bx.W || !al8(op.out)) return bad(at + "DECODEOBB angle view");
        } else if (g.seg || g.obb) {
          return bad(at + (g.seg ? "segment graphs decode with DECODESEG" : "obb graphs decode with DECODEOBB"));
        }
        if (op.stride <= 0) return bad(at + "bad stride");
        if (nlev == 3) return bad(at + "at most 3 detection levels");
        nlev++;
        g.numAnchors += bx.H * bx.W;
        break;
      }
      case MASKS: {
        if (!tenOk(op.a)) return bad(at + "tensor id out of range");
        g.protoTen = op.a;
        g.nm = shp(op.a).C;
        if (!al8(op.a)) return bad(at + "MASKS proto view must be 8-aligned");
        break;
      }
      default:
        return bad(at + "unknown op kind");
    }
  }
  if (g.seg) {
    if (g.protoTen < 0) return bad("segment graph without MASKS op");
    if (g.nm > 64) return bad("at most 64 mask coefficients");
    for (const OpDesc& op : g.ops)
      if (op.kind == DECODESEG && shp(op.out).C != g.nm) return bad("DECODESEG coef count != proto channels");
  }
  if (g.obb && g.protoTen >= 0) return bad("obb graphs carry no MASKS op");
  if (g.cls) {
    // engine/engine.cu:180-190: the probabilities are fetched per image at buffer stride,
    // so they must be a standalone full-width [1,1,nc] buffer
    if (g.probsTen < 0) return bad("classify graph without SOFTMAX");
    if (g.protoTen >= 0) return bad("classify graphs carry no MASKS op");
    const auto& T = g.tens[g.probsTen];
    const auto& Bf = g.bufs[T.buf];
    if (T.coff || T.C != Bf.C || Bf.H != 1 || Bf.W != 1 || T.C != g.nc)
      return bad("probs tensor must be a standalone [1,1,nc] buffer");
  }
  g.detStride = g.obb ? 7 : 6 + (g.seg ? g.nm : 0);
  g.outK = g.obb ? 7 : 6;
  return true;
}

int fuseAdds(std::vector<OpDesc>& ops) {
  std::vector<OpDesc> out;
  int fused = 0;
  for (size_t i = 0; i < ops.size(); i++) {
    OpDesc op = ops[i];
    if (op.kind == CONV && op.b < 0 && i + 1 < ops.size()) {
      const OpDesc& nx = ops[i + 1];
      if (nx.kind == ADD && (nx.a == op.out || nx.b == op.out)) {
        op.b = (nx.a == op.out) ? nx.b : nx.a;
        op.out = nx.out;
        i++;
        fused++;
      }
    }
    out.push_back(op);
  }
  ops.swap(out);
  return fused;
}

}  // namespace yolo
