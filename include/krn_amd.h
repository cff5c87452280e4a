/* krn_amd.h -- C ABI of libkrn_amd.so, the gfx950 (MI355X) kernel library of krn's tile contraction path.
 *
 * Every entry point is host-callable, takes plain device pointers, extents and a hipStream_t passed as void*, enqueues
 * its work on that stream and returns at once. It returns 0 on success and a nonzero code otherwise, leaving a message
 * for krn_amd_last_error(). Tensors are row-major and C-contiguous; bf16 is stored as raw uint16 words, fp8 e4m3fn as
 * uint8 codes (as krn stores them, reference README and tests/compiler/test_tensor_cores.py:305-311).
 *
 * These entry points replace what the reference's AMD route left unbuilt: its HIP renderer emitted the source of a
 * tile kernel (src/krn/compiler/hip.py:20-183) that was compiled only, never loaded or launched, because the backend
 * module `krn.runtime.hip` named by src/krn/runtime/api.py:324 does not exist. A launch there would have gone through
 * hipModuleLaunchKernel with krn's generated-kernel ABI (a tensor is a pointer plus one int64 extent per axis,
 * src/krn/compiler/ir.py:441-452); krn_amd's Python host reaches these entry points through ctypes instead
 * (krn_amd/runtime/library.py), and still uses hipModuleLaunchKernel for tile programs it compiles with hiprtc.
 */
#ifndef KRN_AMD_H
#define KRN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element kinds. */
enum krn_kind { KRN_F32 = 0, KRN_F16 = 1, KRN_BF16 = 2, KRN_F8E4M3 = 3, KRN_I8 = 4, KRN_I32 = 5 };

/* Epilogue operations of krn_gemm_nt, applied in order to the float32 accumulator, each rounded to float32:
 * x * s, x * row[m], x * col[n], x + s, x + row[m], x + col[n], and the activations of krn's lib.matmul epilogues
 * (reference src/krn/lib/lib_kernels.py:31-48 with the formulas of src/krn/compiler/emit.py:112-114):
 * relu x < 0 ? 0 : x, gelu 0.5 x (1 + erf(x / sqrt 2)), silu x / (1 + exp(-x)). A row or column vector is float32
 * unless its operation code adds KRN_VEC_F16 or KRN_VEC_BF16. */
enum krn_epilogue_op {
  KRN_MUL_SCALAR = 0, KRN_MUL_ROW = 1, KRN_MUL_COL = 2, KRN_ADD_SCALAR = 3, KRN_ADD_ROW = 4, KRN_ADD_COL = 5,
  KRN_RELU = 6, KRN_GELU = 7, KRN_SILU = 8, KRN_VEC_F16 = 16, KRN_VEC_BF16 = 32
};

/* C[m, n] = epilogue(sum_k A[m, k] * B[n, k]), A: M x K, B: N x K, C: M x N, all row-major.
 *
 * Replaces the tile program `acc = zeros(f32 | i32, bm, bn); for ks in pipelined(K, bk): acc += a[rows, ks] @
 * b[cols, ks].transpose(); c[rows, cols] = f(acc).to(dtype)` -- krn's Accumulate (reference src/krn/compiler/ir.py:
 * 309-315, capture rule src/krn/compiler/capture.py:3170-3211) lowered by AMDMFMA.product (src/krn/compiler/hip.py:
 * 70-97). in_kind: KRN_BF16 / KRN_F16 (float32 accumulation), KRN_F8E4M3 (float32 accumulation; refused by the
 * reference, src/krn/compiler/matrix.py:129-139) or KRN_I8 (int32 accumulation; refused by the reference capture,
 * src/krn/compiler/capture.py:3193-3201). out_kind: KRN_F32, KRN_F16, KRN_BF16 (round to nearest even), or KRN_I32
 * (int8 operands and no epilogue operations only). ops/scalars/vectors: nops <= 4 epilogue operations; vectors[i]
 * is a device array of length M (row) or N (column), unused for scalar operations and activations. The activations
 * and the bias vector serve krn's lib.matmul kernel (reference src/krn/lib/lib_ours.py:58-75). */
int krn_gemm_nt(int in_kind, const void* a, const void* b, void* c, int out_kind, int64_t m, int64_t n, int64_t k,
                int nops, const int* ops, const float* scalars, const void* const* vectors, void* stream);

/* C[m, n] = epilogue(sum_k A[m, k] * B[k, n]), A: M x K, B: K x N (the NN form), C: M x N, bf16 or f16 operands;
 * out_kind and the epilogue as for krn_gemm_nt. Replaces krn's own GEMM tile program `acc += a[rows, ks] @
 * b[ks, cols]` (reference examples/04_libraries/01_gemm_tiles.py:34-40) and the multiply of lib.matmul
 * (src/krn/lib/lib_kernels.py:31-48), whose B operand is K x N. Products of at least 128 tiles of 256 x 256 with
 * N % 256 == 0, K % 64 == 0, K >= 128 and 16-byte aligned operands read B K-major as it lies and leave `workspace`
 * untouched (it may then be NULL). Any other B is transposed into `workspace` (at least
 * krn_gemm_nn_workspace(n, k) bytes of device memory, owned by the caller) and the NT kernels run on it; the
 * workspace must not be touched by other work until this call's work on `stream` has run. */
int krn_gemm_nn(int in_kind, const void* a, const void* b, void* c, int out_kind, int64_t m, int64_t n, int64_t k,
                int nops, const int* ops, const float* scalars, const void* const* vectors, void* workspace,
                int64_t workspace_bytes, void* stream);

/* Bytes of workspace krn_gemm_nn may need for an N-column, K-row B operand (n * k 16-bit elements; the products
 * that read B as it lies need none). */
int64_t krn_gemm_nn_workspace(int64_t n, int64_t k);

/* Bytes of workspace this krn_gemm_nn call needs: 0 for a product that reads B as it lies (N % 256 == 0,
 * K % 64 == 0, at least 128 tiles of 256 x 256, 16-byte aligned a and b), otherwise krn_gemm_nn_workspace(n, k).
 * Like krn_gemm_nn_workspace, no counterpart in the reference: its NN products need no caller memory. */
int64_t krn_gemm_nn_workspace_for(const void* a, const void* b, int64_t m, int64_t n, int64_t k);

/* krn_gemm_nn without a workspace and without any allocation: the transposed B operand goes to a device array the
 * library holds (64 MiB per GPU it runs on, kept until the process ends; krn_gemm_nn_noalloc_limit() returns the
 * size). This entry point has no counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It calls no hipMalloc,
 * hipFree or allocating library routine; it refuses a B whose n * k * 2 bytes exceed the limit when the product
 * needs the transposed copy (the products krn_gemm_nn reads B as it lies for use no scratch). On a device's first
 * call that uses the array, with the stream's device current, the library looks the array up (hipGetSymbolAddress)
 * and creates one ordering event. The stream must belong to the current device (else an error). Every call on one
 * GPU shares that GPU's array, and the library orders the calls that use it: each eager call makes its stream wait
 * for the event recorded after the previous one, on any stream or host thread. A call on a stream under graph
 * capture is not ordered that way: graph replays and eager calls that overlap on one GPU race, and the caller
 * orders them. */
int krn_gemm_nn_noalloc(int in_kind, const void* a, const void* b, void* c, int out_kind, int64_t m, int64_t n,
                        int64_t k, int nops, const int* ops, const float* scalars, const void* const* vectors,
                        void* stream);

/* Bytes of device scratch krn_gemm_nn_noalloc holds per GPU. */
int64_t krn_gemm_nn_noalloc_limit(void);

/* out (cols x rows) = in (rows x cols) transposed, 16-bit elements: turns the B operand of `a[rows, ks] @ b[ks, cols]`
 * (reference examples/04_libraries/01_gemm_tiles.py:34-40) K-contiguous for krn_gemm_nt. */
int krn_transpose16(const void* in, void* out, int64_t rows, int64_t cols, void* stream);

/* Flash attention forward: O = softmax(scale-scaled Q K^T, causal-masked if asked) V computed with exp2, for tensors
 * (bh, sq, d) / (bh, sk, d) of kind KRN_BF16 or KRN_F16, d = 64 or 128, 16-byte aligned. `scale` multiplies the
 * scores before exp2 (log2(e) / sqrt(d) gives the usual softmax). Replaces krn's flash-attention tile program,
 * reference examples/04_libraries/08_flash_attention.py:35-59 (causal mask `where(k_pos <= q_pos, s, -1e30)`;
 * keys past sk are invalid lanes). One head's keys (sk * d * 2 bytes) and queries rounded up to a whole
 * 256-row tile ((sq + 256) * d * 2 bytes) must each stay under 2 GiB; larger heads are refused with an error. */
int krn_attention_fwd(int kind, const void* q, const void* k, const void* v, void* o, int64_t bh, int64_t sq,
                      int64_t sk, int64_t d, float scale, int causal, void* stream);

/* Row softmax: y[r, c] = exp(x[r, c] - max) / sum exp(x[r, :] - max) over the first `width` columns of each of
 * `rows` rows, float32 arithmetic, one rounding to the element kind (KRN_F32, KRN_F16 or KRN_BF16, the same for x
 * and y). ldx / ldy are the row strides in elements (>= width); columns past width are neither read nor written.
 * Replaces krn's softmax tile programs: the long-row online form, reference examples/02_tiles_and_types/
 * 01_softmax_rows.py:27-40 (column chunks with a running maximum and sum), and the one-tile forms of
 * tests/helpers/example_softmax.py:12-24 (`.softmax(axis=1)`, capture rule src/krn/compiler/capture.py:2883-2917). */
int krn_softmax_rows(int kind, const void* x, void* y, int64_t rows, int64_t width, int64_t ldx, int64_t ldy,
                     void* stream);

/* The message of the calling thread's last failed call. */
const char* krn_amd_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* KRN_AMD_H */
