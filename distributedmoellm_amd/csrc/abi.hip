// Exported C entry points (declared in include/moehip.h): argument checks,
// then the kernels of matvec.hip / dequant.hip / layer.hip.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/moehip.h"
#include "common.h"
#include "blocks.h"
#include "dqgemm.h"
#include "dequant.h"
#include "layer.h"
#include "matvec.h"
#include "prefill.h"
#include "wire.h"

static_assert(sizeof(moe_q4_expert) == sizeof(moe::ExpertDesc), "moe_q4_expert layout");
static_assert(offsetof(moe_q4_expert, xor8) == offsetof(moe::ExpertDesc, xor8), "moe_q4_expert layout");

namespace moe {

static thread_local char g_err[1024];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MOE_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MOE_OK;
}

static hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

#define REQUIRE(cond, ...)                      \
  do {                                          \
    if (!(cond)) return set_error(MOE_EINVAL, __VA_ARGS__); \
  } while (0)

static int check_group_shape(const char* who, int O, int I, int gs) {
  REQUIRE(O > 0 && I > 0, "%s: O=%d and I=%d must be positive", who, O, I);
  REQUIRE(gs > 0 && I % gs == 0, "%s: group size %d must divide I=%d", who, gs, I);
  return MOE_OK;
}

}  // namespace moe

using namespace moe;

MOE_API int moe_version(void) { return 100; }

MOE_API const char* moe_last_error(void) { return g_err; }

MOE_API int moe_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

MOE_API int moe_device_info(int device, char* buf, int len) {
  REQUIRE(buf != nullptr && len > 0, "moe_device_info: no buffer");
  hipDeviceProp_t p;
  const hipError_t e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return set_error(MOE_EHIP, "moe_device_info(%d): %s", device, hipGetErrorString(e));
  snprintf(buf, (size_t)len, "%s|%s|%d|%d|%zu", p.name, p.gcnArchName, p.multiProcessorCount, p.clockRate,
           (size_t)p.totalGlobalMem);
  return MOE_OK;
}

MOE_API int moe_init(int device) {
  const int n = moe_device_count();
  REQUIRE(n > 0, "moe_init: no HIP device is visible");
  REQUIRE(device >= 0 && device < n, "moe_init: device %d of %d", device, n);
  hipDeviceProp_t p;
  const hipError_t e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return set_error(MOE_EHIP, "moe_init(%d): %s", device, hipGetErrorString(e));
  REQUIRE(strncmp(p.gcnArchName, "gfx950", 6) == 0, "moe_init: device %d is %s; these kernels are built for gfx950",
          device, p.gcnArchName);
  return MOE_OK;
}

// ------------------------------------------------------------------ mat-vec

MOE_API int moe_q4_matmul_t(const float* x, int n, const uint8_t* raw, const void* s, int s_f16, int O, int I,
                            int gs, int offset, float* y, void* stream) {
  if (int rc = check_group_shape("moe_q4_matmul_t", O, I, gs)) return rc;
  REQUIRE(I % 2 == 0 && gs % 2 == 0, "moe_q4_matmul_t: I=%d and gs=%d must be even", I, gs);
  REQUIRE(n >= 0, "moe_q4_matmul_t: n=%d", n);
  if (n == 0) return MOE_OK;
  REQUIRE(x && raw && s && y, "moe_q4_matmul_t: null pointer");
  if (n >= kDqRows) {  // many rows: widened in registers, f32 MFMA
    const DqArgs d{x, I, n, raw, s, s_f16, offset ? 0u : 0x88888888u, O, I, gs, y, O};
    if (dq_mfma_ok(DQ_INT4, d)) return run_dq_mfma(DQ_INT4, d, as_stream(stream));
  }
  MVShape sh;
  plan_matvec(FMT_Q4, O, I, gs, &sh);
  MVJob j{};
  j.x = x;
  j.ldx = I;
  j.y = y;
  j.ldy = O;
  j.n = n;
  j.single = MatRef{raw, s, offset ? 0u : 0x88888888u, s_f16};
  return run_matvec(FMT_Q4, sh, j, 1, n, as_stream(stream));
}

MOE_API int moe_q8_matmul_t(const float* x, int n, const int8_t* q, const void* s, int s_f16, int O, int I, int gs,
                            float* y, void* stream) {
  if (int rc = check_group_shape("moe_q8_matmul_t", O, I, gs)) return rc;
  REQUIRE(n >= 0, "moe_q8_matmul_t: n=%d", n);
  if (n == 0) return MOE_OK;
  REQUIRE(x && q && s && y, "moe_q8_matmul_t: null pointer");
  if (n >= kDqRows) {  // many rows: widened in registers, f32 MFMA
    const DqArgs d{x, I, n, q, s, s_f16, 0u, O, I, gs, y, O};
    if (dq_mfma_ok(DQ_INT8, d)) return run_dq_mfma(DQ_INT8, d, as_stream(stream));
  }
  MVShape sh;
  plan_matvec(FMT_Q8, O, I, gs, &sh);
  MVJob j{};
  j.x = x;
  j.ldx = I;
  j.y = y;
  j.ldy = O;
  j.n = n;
  j.single = MatRef{reinterpret_cast<const uint8_t*>(q), s, 0u, s_f16};
  return run_matvec(FMT_Q8, sh, j, 1, n, as_stream(stream));
}

// values per block of a quantized GGUF type, 0 for any other type
static int gguf_block_values(int qtype) {
  int per, size, vals;
  return block_geometry(qtype, &per, &size, &vals) ? per : 0;
}

#define GGUF_TYPES "2 Q4_0, 3 Q4_1, 6 Q5_0, 7 Q5_1, 8 Q8_0, 10 Q2_K, 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K"

MOE_API int moe_gguf_matmul_t(const float* x, int n, const uint8_t* raw, int qtype, int O, int cols, float* y,
                              void* stream) {
  const int blk = gguf_block_values(qtype);
  if (blk == 0) return set_error(MOE_EUNSUPPORTED, "moe_gguf_matmul_t: qtype %d (supported: " GGUF_TYPES ")", qtype);
  REQUIRE(O > 0 && cols > 0 && cols % blk == 0, "moe_gguf_matmul_t: cols=%d must be a positive multiple of %d",
          cols, blk);
  REQUIRE(n >= 0, "moe_gguf_matmul_t: n=%d", n);
  if (n == 0) return MOE_OK;
  REQUIRE(x && raw && y, "moe_gguf_matmul_t: null pointer");
  if ((qtype == FMT_Q8_0 || qtype == FMT_Q4_K) && n >= kDqRows) {  // many rows: blocks widened in registers, f32 MFMA
    const int wf = qtype == FMT_Q8_0 ? DQ_Q8_0 : DQ_Q4_K;
    const DqArgs d{x, cols, n, raw, nullptr, 1, 0u, O, cols, 32, y, O};
    if (dq_mfma_ok(wf, d)) return run_dq_mfma(wf, d, as_stream(stream));
  }
  MVShape sh;
  plan_matvec(qtype, O, cols, blk, &sh);
  MVJob j{};
  j.x = x;
  j.ldx = cols;
  j.y = y;
  j.ldy = O;
  j.n = n;
  j.single = MatRef{raw, nullptr, 0u, 0};
  return run_matvec(qtype, sh, j, 1, n, as_stream(stream));
}

// ------------------------------------------------------------------ dequant

MOE_API int moe_q4_dequant(const uint8_t* raw, const void* s, int s_f16, int O, int I, int gs, int offset,
                           float* out, void* stream) {
  if (int rc = check_group_shape("moe_q4_dequant", O, I, gs)) return rc;
  REQUIRE(I % 2 == 0, "moe_q4_dequant: I=%d must be even", I);
  REQUIRE(raw && s && out, "moe_q4_dequant: null pointer");
  return run_dequant_q4(raw, s, s_f16, O, I, gs, offset ? 0u : 0x88u, out, as_stream(stream));
}

MOE_API int moe_q8_dequant(const int8_t* q, const void* s, int s_f16, int O, int I, int gs, float* out,
                           void* stream) {
  if (int rc = check_group_shape("moe_q8_dequant", O, I, gs)) return rc;
  REQUIRE(q && s && out, "moe_q8_dequant: null pointer");
  return run_dequant_q8(q, s, s_f16, O, I, gs, out, as_stream(stream));
}

MOE_API int moe_gguf_dequant(const uint8_t* raw, int qtype, int O, int cols, float* out, void* stream) {
  const int blk = gguf_block_values(qtype);
  if (blk == 0) return set_error(MOE_EUNSUPPORTED, "moe_gguf_dequant: qtype %d (supported: " GGUF_TYPES ")", qtype);
  REQUIRE(O > 0 && cols > 0 && cols % blk == 0, "moe_gguf_dequant: cols=%d must be a positive multiple of %d", cols,
          blk);
  REQUIRE(raw && out, "moe_gguf_dequant: null pointer");
  return run_dequant_gguf(raw, qtype, O, cols, out, as_stream(stream));
}

// ------------------------------------------------------------------ fused layer

MOE_API size_t moe_q4_layer_workspace(int P, int H, int I) {
  if (P <= 0 || H <= 0 || I <= 0) return 0;
  return q4_layer_workspace(P, H, I);
}

namespace moe {
// the argument checks of moe_q4_layer and moe_q4_layer_noalloc (who: the
// caller's name); fills everything but the workspace. *empty: nothing to do.
static int q4_layer_args(const char* who, const float* x, int ldx, const moe_q4_expert* table, const int* eidx, int k,
                         const int* poff, const int* prow, const float* pw, int P, const int* rrow, const int* rptr,
                         const int* rpair, int nr, float* out, int ldo, int H, int I, int gs, int max_rows,
                         Q4LayerArgs* a, bool* empty) {
  REQUIRE(H > 0 && I > 0 && H % 2 == 0 && I % 2 == 0, "%s: H=%d and I=%d must be positive and even", who, H, I);
  REQUIRE(gs > 0 && gs % 2 == 0 && H % gs == 0 && I % gs == 0, "%s: group size %d must divide H=%d and I=%d", who,
          gs, H, I);
  REQUIRE(k >= 0 && P >= 0 && nr >= 0, "%s: k=%d P=%d nr=%d", who, k, P, nr);
  *empty = k == 0 || P == 0;
  if (*empty) return MOE_OK;
  REQUIRE(max_rows > 0 && max_rows <= P, "%s: max_rows=%d for P=%d", who, max_rows, P);
  REQUIRE(ldx >= H && ldo >= H, "%s: ldx=%d ldo=%d must be >= H=%d", who, ldx, ldo, H);
  REQUIRE(x && table && poff && prow && pw && rrow && rptr && rpair && out, "%s: null pointer", who);
  *a = Q4LayerArgs{};
  a->x = x;
  a->ldx = ldx;
  a->table = reinterpret_cast<const ExpertDesc*>(table);
  a->eidx = eidx;
  a->k = k;
  a->poff = poff;
  a->prow = prow;
  a->pw = pw;
  a->P = P;
  a->rrow = rrow;
  a->rptr = rptr;
  a->rpair = rpair;
  a->nr = nr;
  a->out = out;
  a->ldo = ldo;
  a->H = H;
  a->I = I;
  a->gs = gs;
  a->max_rows = max_rows;
  return MOE_OK;
}
}  // namespace moe

MOE_API int moe_q4_layer(const float* x, int ldx, const moe_q4_expert* table, const int* eidx, int k,
                         const int* poff, const int* prow, const float* pw, int P, const int* rrow, const int* rptr,
                         const int* rpair, int nr, float* out, int ldo, int H, int I, int gs, int max_rows,
                         void* workspace, size_t ws_bytes, void* stream) {
  Q4LayerArgs a;
  bool empty = false;
  if (int rc = q4_layer_args("moe_q4_layer", x, ldx, table, eidx, k, poff, prow, pw, P, rrow, rptr, rpair, nr, out,
                             ldo, H, I, gs, max_rows, &a, &empty))
    return rc;
  if (empty) return MOE_OK;
  const size_t need = q4_layer_workspace(P, H, I);
  if (workspace == nullptr || ws_bytes < need)
    return set_error(MOE_EWORKSPACE, "moe_q4_layer: workspace of %zu bytes, %zu needed", ws_bytes, need);
  REQUIRE(aligned(workspace, 16), "moe_q4_layer: workspace must be 16-byte aligned");
  a.workspace = workspace;
  return run_q4_layer(a, as_stream(stream));
}

MOE_API int moe_q4_layer_noalloc(const float* x, int ldx, const moe_q4_expert* table, const int* eidx, int k,
                                 const int* poff, const int* prow, const float* pw, int P, const int* rrow,
                                 const int* rptr, const int* rpair, int nr, float* out, int ldo, int H, int I, int gs,
                                 int max_rows, void* stream) {
  Q4LayerArgs a;
  bool empty = false;
  if (int rc = q4_layer_args("moe_q4_layer_noalloc", x, ldx, table, eidx, k, poff, prow, pw, P, rrow, rptr, rpair, nr,
                             out, ldo, H, I, gs, max_rows, &a, &empty))
    return rc;
  if (empty) return MOE_OK;
  const size_t need = q4_layer_workspace(P, H, I);
  if (need > kLayerScratchBytes)
    return set_error(MOE_EWORKSPACE,
                     "moe_q4_layer_noalloc: %d pairs at H=%d, I=%d need %zu bytes of scratch, more than the %zu the "
                     "library holds (P * (2I + H) * 4 must not exceed it; use moe_q4_layer with a workspace)",
                     P, H, I, need, kLayerScratchBytes);
  void* ws = nullptr;
  if (int rc = layer_scratch(&ws)) return rc;
  a.workspace = ws;
  return run_q4_layer(a, as_stream(stream));
}

static int check_i8_shape(const char* who, int H, int I, int gs) {
  REQUIRE(H > 0 && I > 0 && gs > 0, "%s: H=%d, I=%d and gs=%d must be positive", who, H, I, gs);
  if (gs % 64 != 0 || gs > 512 || H % gs != 0 || I % gs != 0)
    return set_error(MOE_EUNSUPPORTED, "%s: group size %d must be a multiple of 64 up to 512 dividing H=%d and I=%d",
                     who, gs, H, I);
  return MOE_OK;
}

MOE_API size_t moe_q4_layer_i8_workspace(int P, int H, int I, int gs) {
  if (P <= 0 || H <= 0 || I <= 0 || gs <= 0 || H % gs || I % gs) return 0;
  return q4i8_layer_workspace(P, H, I, gs);
}

MOE_API int moe_q4_layer_i8(const float* x, int ldx, const moe_q4_expert* table, const int* eidx, int k,
                            const int* poff, const int* prow, const float* pw, int P, const int* rrow, const int* rptr,
                            const int* rpair, int nr, float* out, int ldo, int H, int I, int gs, int max_rows,
                            void* workspace, size_t ws_bytes, void* stream) {
  if (int rc = check_i8_shape("moe_q4_layer_i8", H, I, gs)) return rc;
  REQUIRE(k >= 0 && P >= 0 && nr >= 0, "moe_q4_layer_i8: k=%d P=%d nr=%d", k, P, nr);
  if (k == 0 || P == 0) return MOE_OK;
  REQUIRE(max_rows > 0 && max_rows <= P, "moe_q4_layer_i8: max_rows=%d for P=%d", max_rows, P);
  REQUIRE(ldx >= H && ldo >= H, "moe_q4_layer_i8: ldx=%d ldo=%d must be >= H=%d", ldx, ldo, H);
  REQUIRE(x && table && poff && prow && pw && rrow && rptr && rpair && out, "moe_q4_layer_i8: null pointer");
  const size_t need = q4i8_layer_workspace(P, H, I, gs);
  if (workspace == nullptr || ws_bytes < need)
    return set_error(MOE_EWORKSPACE, "moe_q4_layer_i8: workspace of %zu bytes, %zu needed", ws_bytes, need);
  REQUIRE(aligned(workspace, 256), "moe_q4_layer_i8: workspace must be 256-byte aligned");
  Q4LayerArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.table = reinterpret_cast<const ExpertDesc*>(table);
  a.eidx = eidx;
  a.k = k;
  a.poff = poff;
  a.prow = prow;
  a.pw = pw;
  a.P = P;
  a.rrow = rrow;
  a.rptr = rptr;
  a.rpair = rpair;
  a.nr = nr;
  a.out = out;
  a.ldo = ldo;
  a.H = H;
  a.I = I;
  a.gs = gs;
  a.max_rows = max_rows;
  a.workspace = workspace;
  return run_q4i8_layer(a, as_stream(stream));
}

MOE_API int moe_round_q8(const float* x, int ldx, const int* xrow, int n, int K, int gs, int8_t* q, float* d,
                         int32_t* s8, void* stream) {
  REQUIRE(n >= 0 && K > 0 && gs > 0, "moe_round_q8: n=%d K=%d gs=%d", n, K, gs);
  if (gs % 64 != 0 || gs > 512 || K % gs != 0)
    return set_error(MOE_EUNSUPPORTED, "moe_round_q8: group size %d must be a multiple of 64 up to 512 dividing K=%d",
                     gs, K);
  if (n == 0) return MOE_OK;
  REQUIRE(ldx >= K, "moe_round_q8: ldx=%d must be >= K=%d", ldx, K);
  REQUIRE(x && q && d && s8, "moe_round_q8: null pointer");
  return run_round_q8(x, ldx, xrow, n, K, 0, gs, q, d, s8, as_stream(stream));
}

// ------------------------------------------------------------------ wire format

MOE_API int moe_wire_encode(const float* a, int lda, const int* rows, int n, int d, int wire, void* out, float* scale,
                            void* stream) {
  REQUIRE(wire == MOE_WIRE_F32 || wire == MOE_WIRE_F16 || wire == MOE_WIRE_INT8,
          "moe_wire_encode: wire format %d (0 f32, 1 f16, 2 int8)", wire);
  REQUIRE(n >= 0 && d > 0, "moe_wire_encode: n=%d d=%d", n, d);
  if (n == 0) return MOE_OK;
  REQUIRE(lda >= d, "moe_wire_encode: lda=%d must be >= d=%d", lda, d);
  REQUIRE(a && out && (wire != MOE_WIRE_INT8 || scale), "moe_wire_encode: null pointer");
  return run_wire_encode(a, lda, rows, n, d, wire, out, scale, as_stream(stream));
}

MOE_API int moe_wire_decode(const void* in, const float* scale, int wire, int n, int d, const int* rows, float* out,
                            int ldo, void* stream) {
  REQUIRE(wire == MOE_WIRE_F32 || wire == MOE_WIRE_F16 || wire == MOE_WIRE_INT8,
          "moe_wire_decode: wire format %d (0 f32, 1 f16, 2 int8)", wire);
  REQUIRE(n >= 0 && d > 0, "moe_wire_decode: n=%d d=%d", n, d);
  if (n == 0) return MOE_OK;
  REQUIRE(ldo >= d, "moe_wire_decode: ldo=%d must be >= d=%d", ldo, d);
  REQUIRE(in && out && (wire != MOE_WIRE_INT8 || scale), "moe_wire_decode: null pointer");
  return run_wire_decode(in, scale, wire, n, d, rows, out, ldo, as_stream(stream));
}

MOE_API int moe_silu_mul(const float* h, int ldh, int n, int I, float* a, int lda, void* stream) {
  REQUIRE(n >= 0 && I > 0 && ldh >= 2 * I && lda >= I, "moe_silu_mul: n=%d I=%d ldh=%d lda=%d", n, I, ldh, lda);
  if (n == 0) return MOE_OK;
  REQUIRE(h && a, "moe_silu_mul: null pointer");
  return run_silu_mul(h, ldh, n, I, a, lda, as_stream(stream));
}

MOE_API int moe_combine(float* y, int ldy, const float* pw, const int* rrow, const int* rptr, const int* rpair, int nr,
                        int max_pairs, float* out, int ldo, int H, void* stream) {
  REQUIRE(nr >= 0 && H > 0 && ldy >= H && ldo >= H && max_pairs >= 0,
          "moe_combine: nr=%d H=%d ldy=%d ldo=%d max_pairs=%d", nr, H, ldy, ldo, max_pairs);
  if (nr == 0) return MOE_OK;
  REQUIRE(y && pw && rrow && rptr && rpair && out, "moe_combine: null pointer");
  if (max_pairs == 0) return run_combine(y, ldy, pw, rrow, rptr, rpair, nr, out, ldo, H, as_stream(stream));
  return run_combine_runs(y, ldy, pw, rrow, rptr, rpair, nr, max_pairs, out, ldo, H, as_stream(stream));
}

MOE_API int moe_q4_experts_matvec(const float* x, int ldx, const int* xrow, const moe_q4_expert* table,
                                  const int* eidx, int k, const int* poff, int which, int H, int I, int gs,
                                  int max_rows, float* y, int ldy, void* stream) {
  REQUIRE(which == 0 || which == 1, "moe_q4_experts_matvec: which=%d (0 gate|up, 1 down)", which);
  REQUIRE(H > 0 && I > 0 && H % 2 == 0 && I % 2 == 0, "moe_q4_experts_matvec: H=%d and I=%d must be positive and even",
          H, I);
  REQUIRE(gs > 0 && gs % 2 == 0 && H % gs == 0 && I % gs == 0,
          "moe_q4_experts_matvec: group size %d must divide H=%d and I=%d", gs, H, I);
  REQUIRE(k >= 0 && max_rows >= 0, "moe_q4_experts_matvec: k=%d max_rows=%d", k, max_rows);
  if (k == 0 || max_rows == 0) return MOE_OK;
  REQUIRE(x && table && poff && y, "moe_q4_experts_matvec: null pointer");
  const int O = which ? H : 2 * I, cols = which ? I : H;
  REQUIRE(ldx >= (which ? 2 * I : H) && ldy >= O, "moe_q4_experts_matvec: ldx=%d ldy=%d too small", ldx, ldy);
  MVShape sh;
  plan_matvec(FMT_Q4, O, cols, gs, &sh);
  MVJob j{};
  j.x = x;
  j.ldx = ldx;
  j.y = y;
  j.ldy = ldy;
  j.seg = poff;
  j.xrow = xrow;
  j.experts = reinterpret_cast<const ExpertDesc*>(table);
  j.eidx = eidx;
  j.which = which;
  j.half_in = which ? I : 0;
  return run_matvec(FMT_Q4, sh, j, k, max_rows, as_stream(stream));
}

// ------------------------------------------------------------------ prefill

namespace moe {
static size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// largest token count one grouping workgroup takes (its bitsets live in LDS)
// moe_prefill_layer reads a prompt in passes of at most this many tokens (the
// workspace holds one pass)
static constexpr int kPrefillPass = 2048;

struct PrefillWs {
  float* logits;
  int* idx;
  float* w;
  int* eoff;
  int* rows;
  float* wts;
  int* pos;
  int* experts;
  int* offsets;
  int* n_used;
  _Float16* xs;
  float* xf;
  _Float16* act;
  float* af;
  float* y;
  size_t bytes;
};

static PrefillWs prefill_layout(void* base, int T, int E, int k, int H, int I) {
  PrefillWs w{};
  const size_t P = (size_t)T * k;
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t o = off;
    off += align256(n);
    return (char*)base + o;
  };
  w.logits = (float*)take((size_t)router_slices(T, E, H) * T * E * 4);
  w.idx = (int*)take(P * 4);
  w.w = (float*)take(P * 4);
  w.eoff = (int*)take(((size_t)E + 1) * 4);
  w.rows = (int*)take(P * 4);
  w.wts = (float*)take(P * 4);
  w.pos = (int*)take(P * 4);
  w.experts = (int*)take((size_t)E * 4);
  w.offsets = (int*)take(((size_t)E + 1) * 4);
  w.n_used = (int*)take(4);
  w.xs = (_Float16*)take((size_t)T * H * 2);  // the tokens' f16 rows, written by the routing
  w.xf = (float*)take((size_t)T * 4);
  w.act = (_Float16*)take(P * I * 2);
  w.af = (float*)take(P * (I / 16) * 4);
  w.y = (float*)take(P * H * 4);
  w.bytes = off;
  return w;
}

// The expert FFN of grouped rows on the MFMA GEMM, from f16 rows xs with
// factors xf: grouped row q is xs[xrows[q]] (xrows null: xs[q]). act / af take
// silu(gate) * up and its factors (per row and 16 columns); y [P, H] f32.
static int grouped_ffn_f16(const _Float16* xs, const float* xf, const int* xrows, const ExpertDesc* table, int nexp,
                           const int* eoff, int P, int H, int I, int gs, _Float16* act, float* af, float* y, int ldy,
                           hipStream_t st) {
  GemmArgs g{};
  g.A = xs;
  g.lda = H;
  g.xfac = xf;
  g.rows = xrows;
  g.eoff = eoff;
  g.table = table;
  g.which = 0;
  g.K = H;
  g.I = I;
  g.gs = gs;
  g.act = act;
  g.ldact = I;
  g.act_fac = af;
  g.ldaf_out = I / 16;
  if (int rc = run_gemm(MODE_GATE_UP, g, nexp, st)) return rc;
  GemmArgs d{};
  d.A = act;
  d.lda = I;
  d.afac = af;
  d.ldaf = I / 16;
  d.eoff = eoff;
  d.table = table;
  d.which = 1;
  d.K = I;
  d.N = H;
  d.gs = gs;
  d.Y = y;
  d.ldy = ldy;
  (void)P;
  return run_gemm(MODE_DOWN, d, nexp, st);
}

// The same from f32 rows x[rows[q]], gathered into xs / xf (f16) first.
static int grouped_ffn(const float* x, int ldx, const ExpertDesc* table, int nexp, const int* eoff, const int* rows,
                       int P, int H, int I, int gs, _Float16* xs, float* xf, _Float16* act, float* af, float* y,
                       int ldy, hipStream_t st) {
  int rc = run_gather_f16(x, ldx, rows, P, H, xs, xf, st);
  if (rc) return rc;
  return grouped_ffn_f16(xs, xf, nullptr, table, nexp, eoff, P, H, I, gs, act, af, y, ldy, st);
}

// shapes the MFMA tiles do not take are unsupported (not invalid for the format)
static int check_mfma_shape(const char* who, int H, int I, int gs) {
  REQUIRE(H > 0 && I > 0 && gs > 0, "%s: H=%d, I=%d and gs=%d must be positive", who, H, I, gs);
  if (H % 128 != 0 || I % 128 != 0)
    return set_error(MOE_EUNSUPPORTED, "%s: H=%d and I=%d must be multiples of 128", who, H, I);
  // the kernels' group index arithmetic holds for rows below 2^20 columns,
  // their byte offsets for matrices below 4 GiB
  if (H >= (1 << 20) || I >= (1 << 20) || (size_t)H * I >= (1ull << 32))
    return set_error(MOE_EUNSUPPORTED, "%s: H=%d and I=%d must be below 2^20, their product below 2^32", who, H, I);
  if (gs % 32 != 0 || H % gs != 0 || I % gs != 0)
    return set_error(MOE_EUNSUPPORTED, "%s: group size %d must be a multiple of 32 dividing H=%d and I=%d", who, gs,
                     H, I);
  return MOE_OK;
}
}  // namespace moe

MOE_API size_t moe_router_logits_workspace(int T, int E, int H) {
  if (T <= 0 || E <= 0 || H <= 0) return 0;
  return (size_t)router_slices(T, E, H) * T * E * sizeof(float);
}

MOE_API int moe_router_logits(const float* x, int ldx, const float* router, int T, int E, int H, float* logits,
                              void* workspace, size_t ws_bytes, void* stream) {
  REQUIRE(T >= 0 && E > 0 && H > 0 && ldx >= H, "moe_router_logits: T=%d E=%d H=%d ldx=%d", T, E, H, ldx);
  if (T == 0) return MOE_OK;
  REQUIRE(x && router && logits, "moe_router_logits: null pointer");
  // with enough workspace the K dimension is split over more workgroups
  float* scratch = (workspace && ws_bytes >= moe_router_logits_workspace(T, E, H)) ? (float*)workspace : nullptr;
  return run_router_logits(x, ldx, router, T, E, H, logits, scratch, as_stream(stream));
}

MOE_API int moe_route(const float* logits, int T, int E, int k, int normalize, int* idx, float* w, void* stream) {
  REQUIRE(E > 0, "moe_route: E=%d", E);
  REQUIRE(k > 0 && k <= E, "moe_route: k=%d for E=%d", k, E);
  REQUIRE(T >= 0, "moe_route: T=%d", T);
  if (T == 0) return MOE_OK;
  REQUIRE(logits && idx && w, "moe_route: null pointer");
  return run_route(logits, 1, T, E, k, normalize, idx, w, as_stream(stream));
}

MOE_API int moe_group_by_expert(const int* idx, const float* w, int T, int k, int E, int* eoff, int* rows, float* wts,
                                int* pos, int* experts, int* offsets, int* n_used, void* stream) {
  REQUIRE(E > 0 && k > 0 && T >= 0, "moe_group_by_expert: T=%d k=%d E=%d", T, k, E);
  REQUIRE((long)T * k <= (1L << 30), "moe_group_by_expert: %d x %d picks", T, k);
  REQUIRE(idx && w && eoff && rows && wts && pos && experts && offsets && n_used, "moe_group_by_expert: null pointer");
  return run_group(idx, w, T, k, E, eoff, rows, wts, pos, experts, offsets, n_used, as_stream(stream));
}

// the grouped FFN's scratch: gathered rows, their factors, silu(gate) * up and its factors
static size_t ffn_parts(int P, int H, int I, size_t* at) {
  const size_t n[4] = {(size_t)P * H * 2, (size_t)P * 4, (size_t)P * I * 2, (size_t)P * (I / 16) * 4};
  size_t off = 0;
  for (int i = 0; i < 4; ++i) {
    if (at) at[i] = off;
    off += align256(n[i]);
  }
  return off;
}

MOE_API size_t moe_q4_grouped_ffn_workspace(int P, int H, int I) {
  if (P <= 0 || H <= 0 || I <= 0) return 0;
  return ffn_parts(P, H, I, nullptr);
}

MOE_API int moe_q4_grouped_ffn(const float* x, int ldx, const moe_q4_expert* table, int nexp, const int* eoff,
                               const int* rows, int P, int H, int I, int gs, float* y, int ldy, void* workspace,
                               size_t ws_bytes, void* stream) {
  if (int rc = check_mfma_shape("moe_q4_grouped_ffn", H, I, gs)) return rc;
  REQUIRE(nexp >= 0 && P >= 0 && ldx >= H && ldy >= H, "moe_q4_grouped_ffn: nexp=%d P=%d ldx=%d ldy=%d", nexp, P, ldx,
          ldy);
  if (nexp == 0 || P == 0) return MOE_OK;
  REQUIRE(x && table && eoff && rows && y, "moe_q4_grouped_ffn: null pointer");
  REQUIRE(aligned(x, 16) && ldx % 4 == 0, "moe_q4_grouped_ffn: x rows must be 16-byte aligned");
  const size_t need = moe_q4_grouped_ffn_workspace(P, H, I);
  if (!workspace || ws_bytes < need)
    return set_error(MOE_EWORKSPACE, "moe_q4_grouped_ffn: workspace of %zu bytes, %zu needed", ws_bytes, need);
  REQUIRE(aligned(workspace, 256), "moe_q4_grouped_ffn: workspace must be 256-byte aligned");
  size_t at[4];
  ffn_parts(P, H, I, at);
  char* b = (char*)workspace;
  return grouped_ffn(x, ldx, reinterpret_cast<const ExpertDesc*>(table), nexp, eoff, rows, P, H, I, gs,
                     (_Float16*)(b + at[0]), (float*)(b + at[1]), (_Float16*)(b + at[2]), (float*)(b + at[3]), y, ldy,
                     as_stream(stream));
}

MOE_API size_t moe_prefill_workspace(int T, int E, int k, int H, int I) {
  if (T <= 0 || E <= 0 || k <= 0 || H <= 0 || I <= 0) return 0;
  const int pass = T < kPrefillPass ? T : kPrefillPass;
  return prefill_layout(nullptr, pass, E, k, H, I).bytes;
}

MOE_API int moe_prefill_layer(const float* x, int ldx, const float* router, int T, int E, int k, int normalize,
                              const moe_q4_expert* table, int H, int I, int gs, float* out, int ldo, void* workspace,
                              size_t ws_bytes, void* stream) {
  if (int rc = check_mfma_shape("moe_prefill_layer", H, I, gs)) return rc;
  REQUIRE(E > 0 && k > 0 && k <= E, "moe_prefill_layer: E=%d k=%d", E, k);
  if (E > kMaxGridY || k > kCombineMaxPicks)
    return set_error(MOE_EUNSUPPORTED, "moe_prefill_layer: E=%d k=%d (at most %d experts, %d picks a token)", E, k,
                     kMaxGridY, kCombineMaxPicks);
  REQUIRE(T >= 0 && ldx >= H && ldo >= H, "moe_prefill_layer: T=%d ldx=%d ldo=%d", T, ldx, ldo);
  if (T == 0) return MOE_OK;
  REQUIRE(x && router && table && out, "moe_prefill_layer: null pointer");
  REQUIRE(aligned(x, 16) && ldx % 4 == 0, "moe_prefill_layer: x rows must be 16-byte aligned");
  const size_t need = moe_prefill_workspace(T, E, k, H, I);
  if (!workspace || ws_bytes < need)
    return set_error(MOE_EWORKSPACE, "moe_prefill_layer: workspace of %zu bytes, %zu needed", ws_bytes, need);
  REQUIRE(aligned(workspace, 256), "moe_prefill_layer: workspace must be 256-byte aligned");
  hipStream_t st = as_stream(stream);
  const ExpertDesc* tab = reinterpret_cast<const ExpertDesc*>(table);
  const int pass = kPrefillPass;
  for (int t0 = 0; t0 < T; t0 += pass) {  // passes of at most `pass` tokens, as moelan/model.py:640-666
    const int n = T - t0 < pass ? T - t0 : pass;
    PrefillWs w = prefill_layout(workspace, n, E, k, H, I);
    const float* xp = x + (size_t)t0 * ldx;
    int rc, nz = 1;
    if (router_mfma_ok(xp, ldx, router, H)) {
      nz = router_mfma_slices(n, E, H, router_slices(n, E, H));
      rc = run_router_mfma(xp, ldx, router, n, E, H, nz, w.logits, st);
    } else {
      nz = router_slices(n, E, H);
      rc = run_router_partials(xp, ldx, router, n, E, H, nz, w.logits, st);
    }
    // the routing also writes each token's f16 row; grouped row q reads its token's, rows[q]
    if (!rc) rc = run_route(w.logits, nz, n, E, k, normalize, w.idx, w.w, st, xp, ldx, H, w.xs, w.xf);
    if (!rc) rc = run_group(w.idx, w.w, n, k, E, w.eoff, w.rows, w.wts, w.pos, nullptr, nullptr, nullptr, st);
    if (!rc) rc = grouped_ffn_f16(w.xs, w.xf, w.rows, tab, E, w.eoff, n * k, H, I, gs, w.act, w.af, w.y, H, st);
    if (!rc) rc = run_token_combine(w.y, H, w.pos, w.wts, n, k, H, out + (size_t)t0 * ldo, ldo, st);
    if (rc) return rc;
  }
  return MOE_OK;
}

MOE_API int moe_q4_gemm(const float* x, int n, const uint8_t* raw, const void* s, int s_f16, int O, int I, int gs,
                        int offset, float* y, void* stream) {
  REQUIRE(O > 0 && I > 0 && I % 128 == 0, "moe_q4_gemm: O=%d, I=%d must be a multiple of 128", O, I);
  REQUIRE(gs > 0 && gs % 32 == 0 && I % gs == 0, "moe_q4_gemm: group size %d must be a multiple of 32 dividing I=%d",
          gs, I);
  REQUIRE(n >= 0, "moe_q4_gemm: n=%d", n);
  if (I >= (1 << 20) || (size_t)O * I >= (1ull << 33))
    return set_error(MOE_EUNSUPPORTED, "moe_q4_gemm: I=%d must be below 2^20 and the matrix below 4 GiB (O=%d)", I, O);
  if (n == 0) return MOE_OK;
  REQUIRE(x && raw && s && y, "moe_q4_gemm: null pointer");
  REQUIRE(aligned(x, 16), "moe_q4_gemm: x must be 16-byte aligned");
  GemmArgs g{};
  g.rows32 = 1;
  g.X = x;
  g.ldx = I;
  g.rows = nullptr;
  g.table = nullptr;
  g.single = ExpertDesc{raw, s, nullptr, nullptr, offset ? 0u : 0x88u, s_f16};
  g.single_rows = n;
  g.which = 0;
  g.K = I;
  g.N = O;
  g.gs = gs;
  g.Y = y;
  g.ldy = O;
  return run_gemm(MODE_PLAIN, g, 1, as_stream(stream));
}
