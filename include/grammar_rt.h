/* grammar_rt.h -- C ABI of libgrammar_rt.so, the MI355X (gfx950) runtime of
 * the kernel-grammar descent.
 *
 * The reference has no native library: its generated modules are cuTile
 * Python, JIT-compiled by cuda.tile and launched/timed through cupy. Every
 * entry point below replaces one piece of that Python/vendor boundary; the
 * comment on each names the reference site it stands in for.
 *
 * Conventions
 *  - Plain C types only. Device buffers are raw pointers owned by the caller
 *    (PyTorch-ROCm tensors in the Python layer); the library never frees them.
 *  - Every function returns 0 on success or a negative GR_E* code; the
 *    message of the last failure on the calling thread is gr_last_error().
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 */
#ifndef GRAMMAR_RT_H
#define GRAMMAR_RT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define GR_OK 0
#define GR_E_ARG -1       /* invalid argument / unsupported shape */
#define GR_E_COMPILE -2   /* hiprtc compilation failed */
#define GR_E_LOAD -3      /* code object could not be loaded */
#define GR_E_LAUNCH -4    /* kernel launch failed */
#define GR_E_RUNTIME -5   /* any other HIP runtime error */

/* ---- element types ----------------------------------------------------- */
#define GR_F32 0
#define GR_F16 1
#define GR_BF16 2

/* Message describing the last failure on this thread ("" if none). */
const char* gr_last_error(void);

/* Library / toolchain identification, e.g. "gfx950 hiprtc 7.2". The string is
 * part of every on-disk code-object cache key. */
const char* gr_version(void);

/* ---- device properties -------------------------------------------------- */
/* Fills: [0] CU count, [1] max LDS bytes per workgroup, [2] wavefront size,
 * [3] peak engine clock kHz, [4] L2 bytes. For the roofline constants. */
int gr_device_info(int device, long long* out5);

/* ---- compilation (replaces the cuTile JIT: grammar/optimization.py:262-283,
 *      grammar/kernel_ast.py:1228-1229) ------------------------------------ */

/* Compile HIP C++ source `src` with hiprtc for gfx950. Options are passed
 * through (include paths, -D...). On success *code and *code_size receive a
 * malloc'd code object (free with gr_free_code). On a compile error the hiprtc
 * log is copied to `log` (truncated to loglen) and GR_E_COMPILE is returned.
 * Thread-safe: independent programs may be compiled concurrently. No HIP
 * device context is touched. */
int gr_compile(const char* src, const char* name, const char* const* opts, int nopts,
               void** code, size_t* code_size, char* log, size_t loglen);
void gr_free_code(void* code);

typedef struct gr_module gr_module;
typedef struct gr_kernel gr_kernel;

/* Load a code object (from gr_compile or the on-disk cache). */
int gr_module_load(const void* code, size_t code_size, gr_module** out);
void gr_module_free(gr_module* mod);
/* Look up an extern "C" __global__ function by name. The handle lives as long
 * as its module. */
int gr_get_kernel(gr_module* mod, const char* name, gr_kernel** out);

/* ---- launch (replaces ct.launch: grammar/kernel_ast.py:1273-1275) -------- */

/* Launch with every kernel parameter a 64-bit value (device pointers; the
 * renderer bakes every shape into the source). */
int gr_launch(gr_kernel* k, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes,
              void* stream, const uint64_t* args, int nargs);

/* A launch plan: the ordered stage launches of one generated module with
 * their arguments bound (the reference's host fn(*inputs),
 * grammar/kernel_ast.py:1267-1278, minus its per-call cp.zeros allocations:
 * intermediates are allocated once by the caller). */
typedef struct gr_plan gr_plan;
int gr_plan_create(int nsteps, gr_plan** out);
int gr_plan_set_step(gr_plan* p, int i, gr_kernel* k, const uint32_t grid[3], const uint32_t block[3],
                     uint32_t lds_bytes, const uint64_t* args, int nargs);
int gr_plan_run(gr_plan* p, void* stream);
void gr_plan_free(gr_plan* p);

/* ---- timing (replaces cp.cuda.Event timing: grammar/optimization.py:284-300,
 *      bench.py:49-74) ------------------------------------------------------ */
#define GR_TIME_BATCH 0   /* one event pair around `iters` back-to-back runs; mean ms */
#define GR_TIME_MIN 1     /* one event pair per run; minimum ms over `iters` */
/* Each event pair is preceded by a short bounded device spin (about 28 us)
 * that holds the stream while the host enqueues the timed launches, so the
 * time is the GPU's, without the host's launch latency. */
int gr_plan_time(gr_plan* p, void* stream, int warmup, int iters, int mode, float* ms_out);

/* ---- hand-written CDNA4 baselines -------------------------------------- */

/* Flash-style attention forward, O = softmax(scale*Q K^T [causal]) V.
 * Replaces the attention module contract fn(KT, Q, V) (bench.py:14-20,
 * pytorch-naive.py:23-65, grammar/kernel_ast.py:1267-1287) and the SDPA
 * reference point (flash-attn2-sota.py:41-62).
 *  dtype: GR_F16 or GR_BF16 (fp32 accumulate). With GR_F16 the kernel
 *  rounds Q * scale * log2(e) to fp16 once (the scores then need no per-score
 *  scaling); that cannot overflow when scale * log2(e) <= 1 (as for the
 *  default 1/sqrt(D) with D >= 3). A larger fp16 scale (e.g. 1 for a
 *  pre-scaled q) takes kernels that keep Q as given and scale every score,
 *  on one tile only: block_m 64, block_n 32 (0 / 0 pick it; N a multiple of
 *  64). bf16 always keeps Q as given. GR_F32 (the reference's own dtype, fp32
 *  throughout on the fp32 matrix cores): non-causal only, N a multiple of 32,
 *  block_m and block_n ignored (a workgroup owns 32 queries and splits its
 *  keys over its waves); not for gr_attn_fwd_train. When B * H * N / 32 query
 *  blocks would leave CUs idle (N a multiple of 256, at most 128 blocks), the
 *  keys of a query block are also split over 2, 4 or 8 workgroups and a
 *  second launch merges their partials, which sit in a workspace the library
 *  allocates once per (device, stream) and grows on demand: at most
 *  256 * 32 * (D + 2) * 4 bytes (4.3 MB at D = 128), since a split launch has
 *  at most 256 workgroups of 32 queries. A grown buffer is kept until the
 *  process ends, and on the per-thread default stream each host thread keeps
 *  its own. Call once on a stream before capturing such calls into a graph.
 *  Q, V, O: [B, H, N, D] with strides {batch, head, seq} in elements
 *  (unit stride along D). K: [B, H, N, D] if k_transposed == 0, else KT
 *  [B, H, D, N] whose k_strides = {batch, head, d} (unit stride along N).
 *  D in {64, 128}; N a multiple of block_m and block_n.
 *  block_m: queries per workgroup, 64 / 128 / 256 (one wave per 32 queries;
 *  129 / 257: 128 / 256 with the software-pipelined schedule), 0 = the
 *  largest of 256 / 128 / 64 dividing N. block_n: keys per tile, 32 / 64 /
 *  128 (128 at D = 64 only), 0 = 128 at D = 64 when it divides N, else 64
 *  or 32, but 64 where the two-wave body below applies at block_m 256.
 *  fp16 at D = 64, non-causal, 256 x 64 and N a multiple of 256 runs
 *  the kernel with two waves per SIMD and a hand-ordered main loop (160 KiB
 *  of LDS); so does fp16 or bf16 at D = 128 with K transposed, causal or not,
 *  at 256 x 64 and N a multiple of 256 (D = 128 is the default tile there).
 *  Causal grids run each XCD's query blocks longest-first. */
int gr_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H,
                int N, int D, const long long* q_strides, const long long* k_strides,
                const long long* v_strides, const long long* o_strides, int k_transposed,
                int causal, float scale, int block_m, int block_n, void* stream);

/* Training forward: gr_attn_fwd that also writes, per query row, the
 * log-sum-exp of the scaled (masked) scores, natural log, into lse
 * [B*H][N] fp32 (4-byte aligned) for gr_attn_bwd. No counterpart in the
 * reference (forward only); the scope's next-step backward pass. */
int gr_attn_fwd_train(const void* q, const void* k, const void* v, void* o, float* lse, int dtype, int B,
                      int H, int N, int D, const long long* q_strides, const long long* k_strides,
                      const long long* v_strides, const long long* o_strides, int k_transposed, int causal,
                      float scale, int block_m, int block_n, void* stream);

/* Attention backward: dQ, dK, dV of sum(O * dO) for O = softmax(scale Q K^T
 * [causal]) V, from Q, K, V, O, dO and the forward's lse. No counterpart in
 * the reference (forward only); the scope's next-step backward pass.
 *  All nine [B, H, N, D] tensors share `strides` {batch, head, seq} (in
 *  elements, multiples of 8; unit stride along D) and are 16-byte aligned.
 *  D in {64, 128}; N a multiple of 128.
 *  workspace: device memory of gr_attn_bwd_workspace(B, H, N, D) bytes,
 *  16-byte aligned (per-row statistics; the call overwrites it). */
size_t gr_attn_bwd_workspace(int B, int H, int N, int D);
int gr_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                void* dq, void* dk, void* dv, int dtype, int B, int H, int N, int D, const long long* strides,
                int causal, float scale, void* workspace, size_t workspace_bytes, void* stream);

/* Decode-shape attention forward: Nq queries (any count, e.g. 1 for a
 * decode step) against N keys, O = softmax(scale*Q K^T) V, non-causal.
 * No counterpart in the reference, whose attention takes Nq == N
 * (run_attention_search.py:34-114); it is the decode-shape item of the
 * scope's next steps and serves small B*H*Nq, where the query tiles alone
 * cannot fill the GPU.
 *  Q, O: [B, H, Nq, D]; K, V: [B, H, N, D]; strides {batch, head, seq} in
 *  elements (multiples of 8), unit stride along D. N a multiple of 32; D in
 *  {64, 128}; dtype GR_F16 or GR_BF16.
 *  With GR_F16 and more than 4 queries, scale * log2(e) must be <= 1 (as for
 *  gr_attn_fwd; GR_E_ARG otherwise).
 *  Up to 4 queries run on a streaming kernel (K and V read once straight
 *  into registers, scores on the VALU); more on the flash body's MFMA tiles.
 *  splits: workgroups per head (up to 4 queries) or per query tile that
 *  share out the keys (clamped to N/32, or to the number of 64- or 32-key
 *  tiles); with more than one, the partials go
 *  through `workspace` (device memory of at least
 *  gr_attn_decode_workspace(B, H, Nq, D, splits) bytes, 16-byte aligned;
 *  the call then overwrites it) and a second kernel merges them. */
size_t gr_attn_decode_workspace(int B, int H, int Nq, int D, int splits);
int gr_attn_decode(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H, int Nq,
                   int N, int D, const long long* q_strides, const long long* k_strides,
                   const long long* v_strides, const long long* o_strides, float scale, int splits,
                   void* workspace, size_t workspace_bytes, void* stream);

/* gr_attn_decode without any allocation: no counterpart in the reference.
 * For callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc. Same
 * arguments and results as gr_attn_decode minus the workspace: the key-split
 * partials go to a scratch array inside the library, GR_DECODE_SCRATCH_BYTES
 * (16 MiB) per device, held by each device the library runs on until the
 * process ends. A call whose key split needs more than that
 * (gr_attn_decode_workspace(B, H, Nq, D, splits) after the split is clamped)
 * fails with GR_E_ARG before launching anything. Nothing in the array needs
 * to start at zero: every part overwrites its rows before the merge reads
 * them. All calls on one device share its array, so calls that overlap in
 * time on one device (different streams, threads) race: serialise them. */
#define GR_DECODE_SCRATCH_BYTES (16u << 20)
int gr_attn_decode_noalloc(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H, int Nq,
                           int N, int D, const long long* q_strides, const long long* k_strides,
                           const long long* v_strides, const long long* o_strides, float scale, int splits,
                           void* stream);

/* Batched GEMM with fused epilogue, C[z] = act(alpha * A[z] @ B[z]).
 * Replaces the grammar's matmul stage (a stage whose body is matmul over a
 * contraction axis, optionally followed by mulc and relu/silu:
 * grammar/kernel_ast.py:168-223 EMIT_RULES/CONST_OPS, :826-845 accumulator
 * and K loop) as rendered for the MLP (run_mlp_search.py:42-127).
 *  dtype: GR_F16 or GR_BF16 (fp32 accumulate), or GR_F32 (fp32 throughout, on
 *  the fp32 matrix cores: tiles (block_m, block_n) in {32, 64, 128}^2, M and
 *  N multiples of the tile, K a multiple of 8, strides multiples of 4);
 *  batch: number of matrices.
 *  A: [batch][M][K], a_strides = {batch, row}; unit stride along K.
 *  B: [batch][K][N] (b_kmajor == 0, unit stride along N) or [batch][N][K]
 *     (b_kmajor != 0, unit stride along K); b_strides = {batch, row}.
 *  C: [batch][M][N], c_strides = {batch, row}; unit stride along N.
 *  Strides are in elements, multiples of 8 (of 4 for GR_F32); batch stride 0 broadcasts.
 *  epilogue: GR_EPI_NONE, GR_EPI_RELU or GR_EPI_SILU, applied to alpha*acc.
 *  (block_m, block_n) in {(128,128), (256,128), (128,256), (256,256)}
 *  (0 = 256). Any M; N a multiple of 8; K a multiple of 32 (the square
 *  tiles use 64-deep k tiles when K allows). The 256 x 256 tile runs four
 *  waves of 128 x 128 (one per SIMD); the other tiles run eight waves.
 *  With batch 1, a 256 x 256 launch whose last round of workgroups would
 *  fill at most half of the device's CUs is issued as two launches on the
 *  stream: the columns of the whole rounds, then the rest on 256 x 128
 *  tiles (same results: each output's k order is unchanged).
 *  Edge tiles of C are stored only where valid. */
#define GR_EPI_NONE 0
#define GR_EPI_RELU 1
#define GR_EPI_SILU 2
int gr_gemm(const void* a, const void* b, void* c, int dtype, int batch, int M, int N, int K,
            const long long* a_strides, const long long* b_strides, const long long* c_strides,
            int b_kmajor, int epilogue, float alpha, int block_m, int block_n, void* stream);

/* MLP block Y = SiLU(X @ W1) @ W2 as two GEMMs, SiLU fused into the first.
 * The grammar's MLP program (run_mlp_search.py:42-127, with silu in place of
 * relu + residual + LayerNorm). X [M][D], W1 [D][F], W2 [F][D], Y [M][D],
 * all row-major and contiguous; h is caller-provided [M][F] workspace. */
int gr_mlp_fwd(const void* x, const void* w1, const void* w2, void* h, void* y, int dtype, int M,
               int D, int F, int block_m, int block_n, void* stream);

/* Self-test of the 32x32x16 MFMA operand/accumulator layout the kernels
 * assume: one wavefront computes D[32][32] = A[32][16] @ B[16][32] (fp16 in,
 * fp32 out, all row-major device buffers). */
int gr_selftest_mfma32(const void* a, const void* b, float* d, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* GRAMMAR_RT_H */
