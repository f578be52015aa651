// det_hip.h -- C API of det's quantized-linear path on AMD Instinct MI355X (gfx950, HIP).
//
// A drop-in for the GEMM, activation-quantization and runtime entry points of det's CUDA C API (reference
// kernels/cuda/det_cuda.h): the same names, argument meanings and error behaviour, with hipStream_t in place of
// cudaStream_t and det_hip_stream in place of det_cuda_stream.  Conventions of this header:
//   * pointers to tensors live in device memory obtained from det_malloc; det_memcpy moves data to and from the host;
//   * det runs everything on the null stream, in order; det_sync waits for the whole device;
//   * compute entry points return nothing: arguments outside what they accept are reported on stderr and the
//     process aborts, as the reference does.
// Tensors are row-major; element types are fp32 unless a declaration says otherwise.
#pragma once
#include <stdint.h>
#include <stddef.h>
#include <hip/hip_runtime_api.h>
#ifdef __cplusplus
extern "C" {
#endif

// ---- runtime (replaces kernels/cuda/runtime.cu; declarations of det_cuda.h:15-24)
int         det_init(void);                 // selects the current device; 0 on success (called lazily otherwise)
const char* det_device_name(void);
void*       det_malloc(size_t bytes);       // a device block filled with zero bytes, or NULL when none is available
void        det_free(void* p);              // waits for pending work first; aborts on a pointer det_malloc did not return
size_t      det_allocated_bytes(void);      // live det_malloc bytes (the GEMM's own partial-sum buffers not included)
void        det_sync(void);                 // returns once the device is idle; a failed kernel ends the process
void        det_flush(void);                // nothing to do: every launch reaches the device when it is made
void        det_memset(void* p, int value, size_t bytes, hipStream_t st);
void        det_memcpy(void* dst, const void* src, size_t bytes, hipStream_t st);   // any direction (hipMemcpyDefault)
void*       det_hip_stream(void);           // the stream det's work runs on (det_cuda_stream, det_cuda.h:24)

// ---- weights: a quantized linear y = W x, W[N][K] (spec §2; det_cuda.h:27-32)
// Same struct as det_cuda.h.  The pointers hold the HIP layout that det_linear_repack writes (the layout is
// private to this backend, as the Metal backend's tiled codes are to it):
//   wq: packed codes in 64-row tiles, [T][K/128][GB/16][64 rows][16 bytes] with T = 2*ceil(N/128) (whole pairs of
//       tiles), where GB = 128, 96, 64 bytes is one row's packed 128-group (4 * bytes_per_32) for W8, W6, W4; the
//       16-byte chunk c of a tile row is bytes [16c, 16c+16) of that row's packed group, exactly as in the det row;
//       rows past N are zero.  Only when the environment sets DET_PREFILL=streamk (read once per process), the same
//       number of bytes follows: the prefill planes, per 32-row block and 128-group
//       one 16-byte word per lane and plane (4, 3, 2 planes for W8, W6, W4), holding the codes of one row and
//       k-half in the order and scaled packing the M > 64 kernel feeds to the matrix core;
//   c:  [T*64] fp32 (zero past N);
//   m:  [T][K/128][64] uint16 (zero past N).
typedef struct {
    const uint8_t* wq;
    const float*   c;
    const uint16_t* m;
    int N, K, bits;      // bits: 4, 6 or 8
} det_qlinear;

// Sizes of the three planes of det_linear_repack for an N x K linear of `bits`.
// Replaces the row split of the CUDA backend's Backend::linear (reference crates/det/src/cuda.rs:139-163).
void det_linear_sizes(int N, int K, int bits, size_t* wq_bytes, size_t* c_bytes, size_t* m_bytes);
// Load-time repack: `rows` are N det rows ([codes][c fp32][m u16 x K/128], spec/tensor.rs:49-70, the GGUF tensor
// data; several tensors fused along N are simply consecutive rows) in device memory; writes the three planes.
void det_linear_repack(const uint8_t* rows, int N, int K, int bits, uint8_t* wq, float* c, uint16_t* m, hipStream_t st);

// Weight quantizer: N rows of K fp32 weights (device) -> N det rows (device), bit-identical to det convert's
// quantize_rows (reference crates/det/src/quantize.rs:33-100): per 128-group the best of 11 scales by binary64
// squared error, c = f32(max_g s_g / 65535), m_g = rint(s_g / c), wq = rint(w / (c * m_g)).
void det_quantize_rows(const float* w, int N, int K, int bits, uint8_t* rows, hipStream_t st);

// ---- glue (replaces kernels/cuda/norm.cu; det_cuda.h:35-42)
// x[M][n] -> int8 codes xq[M][n] with one fp32 scale per row, sx[M].  Given mx, also one uint16 multiplier per row
// and 128-column group, mx[M][n/128] (then n % 128 == 0): the spec's quant_act_i8g.  mx == NULL: the per-row form
// quant_act_i8.
void det_quant(const float* x, int M, int n, int8_t* xq, float* sx, uint16_t* mx, hipStream_t st);
// RMS-normalise each row of x[M][n] with weights w and eps into y (skipped when y is NULL); when xq is given, the
// normalised rows are also quantized as det_quant does.
void det_rmsnorm_quant(const float* x, const float* w, float eps, int M, int n, float* y, int8_t* xq, float* sx, uint16_t* mx, hipStream_t st);
// silu(g) * u per element into h (skipped when h is NULL), then quantized into hq, sh, mh as det_quant does.
void det_silu_mul_quant(const float* g, const float* u, int M, int n, float* h, int8_t* hq, float* sh, uint16_t* mh, hipStream_t st);

// ---- GEMM (replaces kernels/cuda/gemm.cu; det_cuda.h:45-57)
// For token t and output row n: acc = sum over 128-groups g of m[n][g] * mx[t][g] * (the integer dot product of
// the codes of row n and of token t within g), computed exactly in int64; mx == NULL means every mx is 1.  The
// result is ((float)acc * c[n]) * sx[t], written to y[t][n], or added to it when accumulate is nonzero.  With
// nparts from 2 to 4, the columns are split instead: columns offs[i] .. offs[i+1] - 1 go to dsts[i], a
// [M][offs[i+1] - offs[i]] array (offs[0] must be 0; y is ignored).  M < 1 does nothing.  Aborts with a message for
// K not a multiple of 128, N < 1, more than 4 parts, offs[0] != 0, a NULL y with one part, or bits other than
// 4, 6, 8.
void det_gemm(const det_qlinear* L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, float* y, hipStream_t st);
void det_gemm_ex(const det_qlinear* L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, float* y, int accumulate,
                 int nparts, const int* offs, float* const* dsts, hipStream_t st);
// Scratch contract of det_cuda.h:52-57 (there: per-(token, 128-group) activation sums for W4/W6 with M > 64):
// det_gemm_scratch_bytes(M, K) returns the same size, and det_gemm_set_scratch registers a host-owned buffer (NULL
// unsets).  This backend's kernels need no caller scratch, so the buffer is accepted and left unused.
size_t det_gemm_scratch_bytes(int M, int K);
void det_gemm_set_scratch(void* p, size_t bytes);

// ---- attention (replaces kernels/cuda/attn.cu; det_cuda.h:60-76, cpu.rs:212-285)
typedef struct {
    const float* q_norm;      // [hd]
    const float* k_norm;      // [hd]
    const float* v_scale;     // [n_kv]
    const float* v_inv_scale; // [n_kv]
} det_attn_layer;
// vlo / vhi are kept for the reference's signature (its Metal runtime's V planes); unused here.
typedef struct { int8_t* kq; float* sk; int16_t* vq; int capacity; int8_t* vlo; int8_t* vhi; } det_kv_cache;
// M new tokens at positions pos0 .. pos0 + M - 1: qg[M][n_h][2 hd] (per head q | gate), k, v [M][n_kv][hd], rope
// tables [pos][rot / 2].  Writes the cache rows (kq[pos][n_kv][hd] int8, sk[pos][n_kv], vq[pos][n_kv][hd] int16),
// attends every new token to the positions <= its own, gates by sigmoid(gate) and writes o[M][n_h][hd].
// hd a multiple of 4 up to 1024, n_h a multiple of n_kv, rot even and <= hd, pos0 + M <= capacity, else abort().
// This backend needs no scratch (det_attn_scratch_bytes returns 0; scratch may be NULL).
void det_attention(const det_attn_layer* L, const det_kv_cache* kv, const float* qg, const float* k, const float* v,
                   const float* rope_cos, const float* rope_sin, int rot, float eps,
                   int M, int pos0, int n_h, int n_kv, int hd, float* o, void* scratch, hipStream_t st);
size_t det_attn_scratch_bytes(int M, int n_h, int hd);

// ---- Gated DeltaNet (replaces kernels/cuda/gdn.cu; det_cuda.h:85-98, cpu.rs:287-383)
typedef struct {
    const float* conv;     // [conv_dim][4]
    const float* A;        // [n_v]  (the negated ssm_a of the file)
    const float* dt_bias;  // [n_v]
    const float* norm;     // [dv]
} det_gdn_layer;
typedef struct { float* conv_state; /* [3][conv_dim] oldest first */ float* S; /* [n_v][dk][dv] */ } det_gdn_state;
// qkv[M][conv_dim] (conv_dim = 2 n_k dk + n_v dv), z[M][n_v][dv], a, b [M][n_v]: conv + silu, l2norm of q (times
// QSCALE) and k, the recurrence over the M tokens in order (updating S and the conv window), gated rmsnorm with
// silu(z); writes on[M][n_v][dv].  dk a power of two in 4 .. 128, dv <= 256, n_v a multiple of n_k, scratch of at
// least det_gdn_scratch_bytes(M, ...) bytes, else abort().
void det_gdn(const det_gdn_layer* L, det_gdn_state* S, const float* qkv, const float* z, const float* a, const float* b,
             float eps, int M, int n_k, int n_v, int dk, int dv, float* on, void* scratch, hipStream_t st);
size_t det_gdn_scratch_bytes(int M, int n_k, int n_v, int dk, int dv);

// ---- argmax (replaces det_argmax of runtime.cu; det_cuda.h:43, spec/sample.rs:6-14): out[m] = the lowest index of
// the largest of logits[m][0 .. V)
void det_argmax(const float* logits, int M, int V, int* out, hipStream_t st);

// ---- test hooks (det_test_prim of runtime.cu; det_cuda.h:114-118): the spec's fp32 primitives applied to an array,
// so that tests can compare them bit for bit with the spec.
// Ops by number.  One operand, element by element: exp_f 0, log_f 1, softplus_f 2, sigmoid_f 3, silu_f 4, rint 6,
// reciprocal 7, square root 8, rint then saturating conversion to int32 (stored as fp32) 13.  Two operands,
// element i with element M n - 1 - i: product 9, sum 10, quotient 14, difference 15, spec maximum 16.  Pairs
// (x[2i] low bits, x[2i+1] high bits) read as one int64 and converted to fp32 into out[2i]: by the spec's
// rounding 5, by the compiler's conversion 12.  The spec's pairwise tree sum of each row of n into out[row]: 11.
void det_test_prim(int op, const float* x, int M, int n, float* out, hipStream_t st);
// Test hooks of the model runner's one-token FFN path (no det_cuda.h counterpart; for tests of this library):
//   det_test_gemv_silu0: det_gemm_ex with M = 1 and Parts output (2 to 4 parts from column 0), storing silu_f(v)
//     instead of v for the columns of part 0 (the gate half of a fused gate|up linear);
//   det_test_mul_quant: h = a * b per element, quantized in group mode (n % 128 == 0, n <= 32768): with a = silu_f(g)
//     the same codes and scales as det_silu_mul_quant(g, b).  Other shapes abort.
void det_test_gemv_silu0(const det_qlinear* L, const int8_t* xq, const float* sx, const uint16_t* mx, int nparts,
                         const int* offs, float* const* dsts, hipStream_t st);
void det_test_mul_quant(const float* a, const float* b, int M, int n, int8_t* xq, float* sx, uint16_t* mx, hipStream_t st);
// Test hook for measurement (no det_cuda.h counterpart): a plain streaming read of `bytes` (a multiple of 16) of
// device memory by `blocks` workgroups, each storing the xor of its contiguous share into sink[block]; bench.py
// times it as the floor a single-pass read of a GEMV's weight bytes can reach.
void det_test_read(const void* p, size_t bytes, int blocks, unsigned* sink, hipStream_t st);

#ifdef __cplusplus
}
#endif
