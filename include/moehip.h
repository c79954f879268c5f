/*
 * moehip: MI355X (gfx950) routed-expert compute path of moelan, as a C ABI.
 *
 * Every pointer named a "device" pointer is HBM memory of the current HIP
 * device (e.g. a torch tensor's data_ptr()); host pointers are marked as such.
 * `stream` is a hipStream_t (NULL: the default stream). Calls are stream
 * ordered and return before the GPU finishes. Every call returns 0 on success
 * or a non-zero MOE_E* code, with a message in moe_last_error() (per thread).
 * The library allocates nothing: scratch comes from the caller's workspace.
 *
 * Conventions shared with moelan (citations are files of the reference):
 *   int4 "Packed4"  raw uint8 [O, I/2], byte j = column 2j (low nibble) and
 *                   2j+1 (high nibble), two's-complement nibbles; offset != 0
 *                   means the bytes were XOR-ed with 0x88 already (u = v + 8).
 *                   Scales [O, I/gs], f32 or f16 (s_f16 != 0).
 *                   moelan/experts.py:170-236, moelan/tiny.py:94-106
 *   int8 "GroupQuant" q int8 [O, I], scales [O, I/gs]. moelan/experts.py:125-167
 *   GGUF            raw uint8 [O, row bytes], a quantized ggml type: 2 Q4_0,
 *                   3 Q4_1, 6 Q5_0, 7 Q5_1, 8 Q8_0, 10 Q2_K, 11 Q3_K, 12 Q4_K,
 *                   13 Q5_K, 14 Q6_K. moelan/gguf.py:36-42, moelan/kernels.py:262-476
 */
#ifndef MOEHIP_H
#define MOEHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_OK 0
#define MOE_EINVAL 1
#define MOE_EHIP 2
#define MOE_EWORKSPACE 3
#define MOE_EUNSUPPORTED 4

/* ---------------------------------------------------------------- library */

/* Checks that `device` is usable (gfx950 class, MFMA present).
 * Replaces the import-time probe that sets ENABLED / WHY_DISABLED,
 * moelan/kernels.py:19-41. */
int moe_init(int device);

/* Message of the last failed call on this thread ("" if none).
 * moelan/kernels.py:20 (WHY_DISABLED). */
const char* moe_last_error(void);

/* Number of visible HIP devices (0 without a GPU); never fails. */
int moe_device_count(void);

/* "name|arch|CUs|max clock kHz|HBM bytes" of `device` into buf. */
int moe_device_info(int device, char* buf, int len);

/* ABI version (major*100 + minor). */
int moe_version(void);

/* ------------------------------------------------------- one matrix: x @ W.T */

/* y[n, O] = x[n, I] @ W.T for colibri int4 weights, f32 accumulate.
 * Replaces q4_matmul_t(x, raw, s, gs, offset), moelan/kernels.py:1018-1027
 * (kernels _q4 :85-106 and _q4_rows :108-131). x, raw, s, y: device.
 * Numerics (this call, moe_q4_experts_matvec and moe_q4_layer): on the
 * chunked kernels (rows cut into 16- or 24-byte chunks, which covers the
 * usual expert shapes) each run of 32 (or 16) activations is taken as exact
 * fixed point rint(x * 2^S), S set by the run's largest |x|, and multiplied
 * with the nibbles exactly (integer dot products), then scaled by the group
 * scale in f32. Each product term is off by at most 8 * 2^-22 of that
 * largest |x| (so a run holding an outlier 2^k times its other values keeps
 * about 22 - k bits of them); an Inf or NaN in x makes the outputs that use
 * it NaN.
 * Other shapes multiply in f32. */
int moe_q4_matmul_t(const float* x, int n, const uint8_t* raw, const void* s, int s_f16, int O, int I, int gs,
                    int offset, float* y, void* stream);

/* y[n, O] = x @ W.T for group-scaled int8 weights.
 * Replaces q8_matmul_t(x, q, s, gs), moelan/kernels.py:1030-1032 (_q8 :152-168,
 * _q8_rows :133-150). */
int moe_q8_matmul_t(const float* x, int n, const int8_t* q, const void* s, int s_f16, int O, int I, int gs,
                    float* y, void* stream);

/* y[n, O] = x[n, cols] @ W.T for GGUF block-quantized rows of any quantized
 * type, any cols (rows past 8192 values take one launch per 8192-value
 * segment, summed in segment order); rows need no alignment.
 * Replaces gguf_matmul_t(x, raw, qtype, cols), moelan/kernels.py:981-998
 * (_mv_q8_0 :482-498, _mv_q4_k :499-528, _mv_q5_k :529-561, _mv_q6_k
 * :562-596, _mv_q2_k :597-632, _mv_q3_k :642-677, _gguf_mm :678-691). */
int moe_gguf_matmul_t(const float* x, int n, const uint8_t* raw, int qtype, int O, int cols, float* y,
                      void* stream);

/* ---------------------------------------------------------------- dequant */

/* out[O, I] f32 = (u - 8) * s, bit-exact.
 * Replaces q4_dequant(raw, s, gs, offset, out), moelan/kernels.py:971-973. */
int moe_q4_dequant(const uint8_t* raw, const void* s, int s_f16, int O, int I, int gs, int offset, float* out,
                   void* stream);

/* out = q * s, bit-exact. Replaces q8_dequant, moelan/kernels.py:976-978. */
int moe_q8_dequant(const int8_t* q, const void* s, int s_f16, int O, int I, int gs, float* out, void* stream);

/* out[O, cols] f32 from GGUF rows, bit-exact with the reference decoders.
 * Replaces gguf_dequant(raw, qtype, out), moelan/kernels.py:1001-1003. */
int moe_gguf_dequant(const uint8_t* raw, int qtype, int O, int cols, float* out, void* stream);

/* a[n, I] = silu(h[:, :I]) * h[:, I:] for h [n, 2I] (row strides ldh, lda).
 * The middle of Expert.__call__, moelan/experts.py:256-259 (silu :62-63). */
int moe_silu_mul(const float* h, int ldh, int n, int I, float* a, int lda, void* stream);

/* out[rrow[i]] += sum over q in rptr[i]..rptr[i+1] of pw[p] * y[p], p = rpair[q]:
 * the weighted combine of per-expert outputs, out[rows] += e(x[rows]) * w,
 * moelan/experts.py:648-651, 707-727 and moelan/kernels.py:778-782, 968.
 * Summed in a fixed order (64 strided partial sums, each in list order, added
 * by a fixed binary tree), so results repeat bit for bit; no atomics. y [P, H]
 * (stride ldy) is only read. max_pairs (an upper bound of a row's pairs, or 0)
 * is accepted and not needed. out stride ldo. */
int moe_combine(float* y, int ldy, const float* pw, const int* rrow, const int* rptr, const int* rpair, int nr,
                int max_pairs, float* out, int ldo, int H, void* stream);

/* -------------------------------------------- one MoE layer, few rows each */

/* One int4 expert: what q4_expert_ptrs() returns, moelan/kernels.py:929-939
 * (four addresses and the XOR), plus the scale type. */
typedef struct moe_q4_expert {
  const void* gu_w; /* gate|up bytes [2I, H/2] */
  const void* gu_s; /* scales [2I, H/gs] */
  const void* dn_w; /* down bytes [H, I/2] */
  const void* dn_s; /* scales [H, I/gs] */
  uint32_t xor8;    /* 0x88 for stored two's-complement nibbles, 0 for XOR-ed copies */
  int32_t s_f16;    /* scales are f16 */
} moe_q4_expert;

/* Bytes of workspace moe_q4_layer needs for P pairs. */
size_t moe_q4_layer_workspace(int P, int H, int I);

/* out[r] += sum over pairs p of row r of pw[p] * expert(x[r]), for k experts
 * given as table[eidx[m]] (eidx NULL: table[m]) with pairs poff[m]..poff[m+1]
 * (poff ascending from poff[0] = 0 to poff[k] = P; input rows prow[p], gate
 * weights pw[p]). Rows touched: rrow[0..nr), whose
 * pairs are rpair[rptr[i]..rptr[i+1]] in ascending order; each row's sum is
 * formed in a fixed order (as moe_combine) and then added to out, as the
 * reference does.
 * max_rows: the largest poff[m+1]-poff[m]. All arrays: device.
 * Replaces moe_q4(x, items, H, I, gs, out), moelan/kernels.py:942-968
 * (_moe_q4 :712-782, float activations). */
int moe_q4_layer(const float* x, int ldx, const moe_q4_expert* table, const int* eidx, int k, const int* poff,
                 const int* prow, const float* pw, int P, const int* rrow, const int* rptr, const int* rpair, int nr,
                 float* out, int ldo, int H, int I, int gs, int max_rows, void* workspace, size_t ws_bytes,
                 void* stream);

/* moe_q4_layer with no workspace argument: the call's scratch (what
 * moe_q4_layer would take from its workspace: the gate|up outputs h [P, 2I] and
 * down outputs y [P, H], f32, and for experts with several rows their
 * activation limbs) lives in 32 MiB of device memory the library holds on
 * each device it runs on, from the first call there until the process ends,
 * so the call allocates nothing. It has no counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Limit:
 * moe_q4_layer_workspace(P, H, I) <= 32 MiB (about 59 KB a pair at H=2048,
 * I=768: 564 pairs; about 119 KB at H=4096, I=1536: 282 pairs), else
 * MOE_EWORKSPACE. Every call on one device shares that device's scratch:
 * calls that overlap on a device (other streams, other threads) race. Same
 * arguments, results and numerics as moe_q4_layer. */
int moe_q4_layer_noalloc(const float* x, int ldx, const moe_q4_expert* table, const int* eidx, int k,
                         const int* poff, const int* prow, const float* pw, int P, const int* rrow, const int* rptr,
                         const int* rpair, int nr, float* out, int ldo, int H, int I, int gs, int max_rows,
                         void* stream);

/* One sweep of the layer call over its experts' matrices: for expert
 * table[eidx[m]] (eidx NULL: table[m]) and its pairs p in poff[m]..poff[m+1],
 * y[p] = xin(p) @ W.T where W is the gate|up matrix (which = 0; xin(p) = x row
 * xrow[p], or row p when xrow is NULL) or the down matrix (which = 1; xin(p)
 * = silu(h[:, :I]) * h[:, I:] of row p of x = h, the gate|up outputs).
 * The gate|up and down phases of _moe_q4, moelan/kernels.py:727-745, 749-777. */
int moe_q4_experts_matvec(const float* x, int ldx, const int* xrow, const moe_q4_expert* table, const int* eidx,
                          int k, const int* poff, int which, int H, int I, int gs, int max_rows, float* y, int ldy,
                          void* stream);

/* ------------------------------------- the same call, int8 activations */

/* Bytes of workspace moe_q4_layer_i8 needs for P pairs. */
size_t moe_q4_layer_i8_workspace(int P, int H, int I, int gs);

/* moe_q4_layer with the activations rounded to int8 per group of gs (a
 * multiple of 64 up to 512, dividing H and I): each input row (once, however
 * many pairs read it), and each pair's SiLU(gate)*up row, rounded as _round_q8; each group's product an exact integer sum of
 * unsigned nibble * int8, added as f32(isum - 8*sum q) * (s_w * d); the same
 * combine. The reference's int8-activation layer call: moe_q4 when
 * int8_act_for(H, I, gs) holds, moelan/kernels.py:942-968 (_moe_q4i :854-917,
 * _round_q8 :833-852, _q4c64 :807-831). Workspace 256-byte aligned. */
int moe_q4_layer_i8(const float* x, int ldx, const moe_q4_expert* table, const int* eidx, int k, const int* poff,
                    const int* prow, const float* pw, int P, const int* rrow, const int* rptr, const int* rpair, int nr,
                    float* out, int ldo, int H, int I, int gs, int max_rows, void* workspace, size_t ws_bytes,
                    void* stream);

/* Rows xrow[i] (xrow NULL: i) of x [*, ldx], i < n, rounded to int8 per group
 * of gs (a multiple of 64 up to 512) as _round_q8, moelan/kernels.py:833-852: scale d = max|v| / 127 (1 for
 * a zero group), q = floor(v * (1/d) + 0.5), s8 = 8 * the group's sum of q.
 * q [n, K] bytes, each 32-column chunk as its 16 even columns then its 16 odd
 * ones (the reference's qe / qo halves); d, s8 [n, K/gs]. All device arrays. */
int moe_round_q8(const float* x, int ldx, const int* xrow, int n, int K, int gs, int8_t* q, float* d, int32_t* s8,
                 void* stream);

/* ------------------------------------------------------------ wire format */

/* Activations between a coordinator and its workers (moelan/protocol.py:90-123). */
#define MOE_WIRE_F32 0
#define MOE_WIRE_F16 1
#define MOE_WIRE_INT8 2

/* Rows rows[r] (rows NULL: r) of a [*, lda], r < n, encoded as encode_rows
 * (moelan/protocol.py:99-114) into out [n, d]: f32 (a copy), f16 (round to
 * nearest even, as numpy's astype), or int8 with scale [n, d/gs] f32, gs = 64
 * when 64 divides d, else d: s = max|g| / 127 (1 for a zero group),
 * q = clip(rint(g / s), -127, 127). Bit-exact for finite inputs. The worker
 * encodes y[touched] this way (moelan/worker.py:352-354). */
int moe_wire_encode(const float* a, int lda, const int* rows, int n, int d, int wire, void* out, float* scale,
                    void* stream);

/* Row r of in [n, d] decoded (decode_rows, moelan/protocol.py:116-123: q * s
 * for int8) into out[rows[r]] (rows NULL: out[r]), row stride ldo. */
int moe_wire_decode(const void* in, const float* scale, int wire, int n, int d, const int* rows, float* out, int ldo,
                    void* stream);

/* ------------------------------------------------ prompt reading (prefill) */

/* Bytes of workspace that let moe_router_logits split H over more workgroups. */
size_t moe_router_logits_workspace(int T, int E, int H);

/* logits[T, E] = x[T, H] @ router[E, H].T in f32 (the router product of
 * MoEModel._ffn, moelan/model.py:597). Workspace optional (NULL: one slice). */
int moe_router_logits(const float* x, int ldx, const float* router, int T, int E, int H, float* logits,
                      void* workspace, size_t ws_bytes, void* stream);

/* Softmax router with top-k: idx[T, k] int32, w[T, k] f32, largest first,
 * ties to the lower expert id, NaN probabilities last; w divided by its sum
 * (numpy's pairwise summation order) when normalize != 0. Any E, 1 <= k <= E.
 * Replaces route(), moelan/model.py:154-167 (softmax :83-86). */
int moe_route(const float* logits, int T, int E, int k, int normalize, int* idx, float* w, void* stream);

/* Stable grouping of the T*k picks by expert, as group_by_expert(),
 * moelan/model.py:226-236: experts[0..*n_used) ascending with their pick
 * ranges offsets[0..*n_used]; eoff[E+1] the same ranges for every expert id;
 * rows[q] / wts[q] the token and weight of grouped pick q; pos[t*k+j] where
 * pick j of token t went (-1 for an expert id outside 0..E-1). All device
 * arrays. */
int moe_group_by_expert(const int* idx, const float* w, int T, int k, int E, int* eoff, int* rows, float* wts, int* pos,
                        int* experts, int* offsets, int* n_used, void* stream);

/* Bytes of workspace moe_q4_grouped_ffn needs for P grouped rows. */
size_t moe_q4_grouped_ffn_workspace(int P, int H, int I);

/* y[q] = expert_e(x[rows[q]]) for every grouped row q of every expert e
 * (rows eoff[e] .. eoff[e+1], expert table[e]): the SwiGLU expert FFN of
 * Expert.__call__, moelan/experts.py:256-259, on many rows at once, as the
 * reference's big-group path (dequant + BLAS, moelan/experts.py:216-219,
 * 718-723). int4 -> f16 in registers, f16 MFMA with f32 accumulation
 * (relative error ~1e-3 at most). H, I multiples of 128; gs a multiple of 32;
 * nexp <= 65535. */
int moe_q4_grouped_ffn(const float* x, int ldx, const moe_q4_expert* table, int nexp, const int* eoff, const int* rows,
                       int P, int H, int I, int gs, float* y, int ldy, void* workspace, size_t ws_bytes, void* stream);

/* Bytes of workspace moe_prefill_layer needs (one pass of at most 2048 tokens). */
size_t moe_prefill_workspace(int T, int E, int k, int H, int I);

/* One MoE layer over T tokens: router logits, route, group, grouped expert
 * FFN, weighted combine; out[t] = sum over t's k experts (ascending id) of
 * w * expert(x[t]) (written, not added). table[e] is expert e of the layer.
 * MoEModel._ffn + LocalBackend._moe + ExpertStore.compute for a prompt,
 * moelan/model.py:597-606, 274-278, moelan/experts.py:641-670.
 * E <= 65535 experts, k <= 4096 picks a token. */
int moe_prefill_layer(const float* x, int ldx, const float* router, int T, int E, int k, int normalize,
                      const moe_q4_expert* table, int H, int I, int gs, float* out, int ldo, void* workspace,
                      size_t ws_bytes, void* stream);

/* y[n, O] = x[n, I] @ W.T for one int4 matrix on many rows through the f16
 * MFMA path (Packed4.matmul_t's BLAS branch, moelan/experts.py:216-219);
 * x 16-byte aligned. */
int moe_q4_gemm(const float* x, int n, const uint8_t* raw, const void* s, int s_f16, int O, int I, int gs, int offset,
                float* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOEHIP_H */
