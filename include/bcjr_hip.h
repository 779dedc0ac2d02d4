/*
 * bcjr_hip.h -- C ABI of the MI355X (gfx950) BCJR forward-backward engine.
 *
 * This is the drop-in boundary for the differentiable trellis-coded quantizer's
 * soft-quantization node and its T->0 Viterbi mode.  Each entry point replaces
 * the compute inside one reference interface (file:line into the reference
 * repository), keeping its argument meaning and tensor layout:
 *
 *   bcjr_forward   src/bcjr/forward_backward.py:190-232   bcjr_forward_backward
 *                  (soft codewords + log Z; also the forward of
 *                  src/bcjr/bcjr_monolithic.py:161-189)
 *   bcjr_forward_internals  the return_internals=True branch,
 *                  src/bcjr/forward_backward.py:230-231
 *   bcjr_backward  src/bcjr/bcjr_monolithic.py:192-243   analytic backward of the node
 *                  (eager autograd of forward_backward.py:106-232)
 *   bcjr_viterbi   src/viterbi/cuda_kernel.py:166-220    viterbi_encode_v_batched_cuda,
 *                  with the tie rules of src/viterbi/encode.py:250-307
 *   bcjr_viterbi_constrained  src/viterbi/encode.py:105-172, 328-389
 *                  (viterbi_encode_constrained, _v: the inner pass of tail-biting)
 *   bcjr_viterbi_trace  src/viterbi/encode.py:250-307 with return_trace=True
 *                  (trace_err and backpointers of viterbi_encode_v)
 *   bcjr_decode    src/viterbi/encode.py:310-325 (viterbi_decode_v) and
 *                  src/qat/ste.py:270-283 (_replay_walks)
 *   bcjr_dequant   src/quantize/serialize.py:56-107 (dequant_target, before the
 *                  inverse RHT) and src/quantize/lut_ft.py:59-79
 *   bcjr_codebook  src/codes/ref.py:33-41,76-91 (1MAD, 3INST) and
 *                  src/qat/ste.py:376-392 (make_hyb_codebook_gpu)
 *   bcjr_hadamard  fast_hadamard_transform.hadamard_transform (src/rht/transform.py:44-55)
 *   bcjr_rht       src/qat/ste.py:113-135 (apply_rht_gpu, apply_inverse_rht_gpu),
 *                  src/rht/transform.py:65-126
 *   bcjr_rht_batched  the per-expert RHT calls of src/qat/qat_moe_layer.py:106-114,
 *                  in one launch pair
 *
 * Conventions
 *   - All pointers are device pointers owned by the caller; inputs are read-only.
 *   - Layouts are the reference's: sequences (B, N, V) row-major float32 with
 *     N = steps and V = weights per step; codebook (2^L, V) float32; HYB LUT
 *     (2^Q, 2) float32.  bitstream/walk (B, N) int32; start_state (B,) int32.
 *   - Work is enqueued on `stream` and is stream-ordered: no host synchronisation,
 *     no allocation, so the calls can be captured into a HIP graph.  Scratch
 *     memory is the caller's `ws` buffer of at least bcjr_workspace_bytes() bytes.
 *   - Every entry point returns 0 on success or a negative BCJR_E* status;
 *     bcjr_strerror() names it and bcjr_last_error() gives the detail of the
 *     calling thread's last failure.  No C++ exception crosses the ABI.
 *   - Temperature T is read from device memory (a 0-d tensor or one value per
 *     sequence when t_per_seq != 0); it must be finite and > 0.  The soft
 *     kernels check this on the device: a sequence whose T is not finite and
 *     positive, or whose weights (or, for the backward, upstream gradients) are
 *     not all finite, gets NaN in every output of that sequence (soft and log Z,
 *     or its gradient); the other sequences of the launch are unaffected.
 *   - Calls on different streams may overlap as long as their `ws` buffers
 *     differ.
 */
#ifndef BCJR_HIP_H_
#define BCJR_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

/* Codebook sources (c(s) for state s). */
enum {
    BCJR_CODE_TABLE = 0,  /* explicit (2^L, V) float32 table                   */
    BCJR_CODE_1MAD = 1,   /* LCG + byte sum, V = 1 (src/codes/ref.py:33-41)     */
    BCJR_CODE_3INST = 2,  /* LCG + fp16 pair, V = 1 (src/codes/ref.py:76-91)    */
    BCJR_CODE_HYB = 3     /* x*x+x hash into a (2^Q, 2) LUT, V = 2              */
};

/* Operations, for bcjr_workspace_bytes(). */
enum { BCJR_OP_FORWARD = 0, BCJR_OP_BACKWARD = 1, BCJR_OP_VITERBI = 2 };

/* Status codes. */
enum {
    BCJR_OK = 0,
    BCJR_EINVAL = -1,       /* bad argument (shape, null pointer, code/V mismatch) */
    BCJR_EUNSUPPORTED = -2, /* (L, k, V) combination not built                     */
    BCJR_EWORKSPACE = -3,   /* workspace smaller than one sequence slot            */
    BCJR_EHIP = -4          /* HIP runtime error (launch, attribute, device query) */
};

/* Problem description.  kV = k * V bits per step must be 1, 2 or 4, and
 * 2*kV <= L <= 16 (kV = 1 requires L <= 11 and the table code). */
typedef struct {
    int L;          /* state bits: S = 2^L states                          */
    int k;          /* bits per weight                                     */
    int V;          /* weights per step (vector dimension), 1 or 2         */
    int64_t B;      /* number of sequences (tiles)                         */
    int64_t N;      /* steps per sequence (sequence length / V), <= 4096   */
    int code;       /* BCJR_CODE_*                                         */
    int Q;          /* HYB LUT bits (2^Q rows), 1..12; ignored otherwise   */
    int t_per_seq;  /* 0: T is one value; 1: T holds B values              */
} bcjr_problem;

/* Bytes of device workspace the operation wants for this problem on the
 * current device.  A smaller buffer (>= one sequence slot) also works, with
 * fewer sequences in flight. */
int bcjr_workspace_bytes(const bcjr_problem* prob, int op, size_t* bytes);

/* Soft codewords E_P[c(s_t)] (B, N, V) and log Z (B,) (natural log, including
 * the free-start factor 2^kV of forward_backward.py:143).  logZ may be NULL.
 * Replaces bcjr_forward_backward (src/bcjr/forward_backward.py:190-232). */
int bcjr_forward(const bcjr_problem* prob, const float* seq, const float* T,
                 const float* codebook_or_lut, float* soft, float* logZ,
                 void* ws, size_t ws_bytes, hipStream_t stream);

/* bcjr_forward plus the diagnostics of return_internals=True
 * (src/bcjr/forward_backward.py:230-231): marginals P (B, N, 2^L), log_alpha and
 * log_beta (B, N, 2^L), natural log, as the reference defines them
 * (log_alpha_{-1} = 0, log_beta_{N-1} = 0).  Meant for small B (the reference
 * uses it on <= 32 tiles, src/bcjr/anneal.py:143-184). */
int bcjr_forward_internals(const bcjr_problem* prob, const float* seq, const float* T,
                           const float* codebook_or_lut, float* soft, float* logZ,
                           float* marginals, float* log_alpha, float* log_beta,
                           void* ws, size_t ws_bytes, hipStream_t stream);

/* bcjr_forward plus the marginal entropy of every step, entropy (B, N) float32,
 * H_t = -sum_s P_t(s) ln P_t(s) in nats, accumulated inside the beta sweep: no
 * (B, N, 2^L) tensor is formed, so it runs on whole layers at about the cost of
 * bcjr_forward.  Replaces the P-materialising body of entropy_diagnostic
 * (src/bcjr/anneal.py:143-184, which calls forward_backward.py:190-232 with
 * return_internals=True and reduces -(P * log P).sum(-1)). */
int bcjr_forward_entropy(const bcjr_problem* prob, const float* seq, const float* T,
                         const float* codebook_or_lut, float* soft, float* logZ, float* entropy,
                         void* ws, size_t ws_bytes, hipStream_t stream);

/* bcjr_forward without a workspace argument: it allocates nothing.  No
 * counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The sequence slots live in a static device array of
 * BCJR_NOALLOC_SCRATCH_BYTES (128 MiB) that the library holds on every GPU it
 * runs on until the process ends; as many sequences are in flight as slots fit
 * (8 at L=16, kV=2, N=256), so its throughput is below bcjr_forward's.  A
 * problem whose one slot (N * 2^(L-kV) * 4 bytes) exceeds the array returns
 * BCJR_EWORKSPACE.  Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race and must be
 * serialised by the caller.  The first call on a device looks up the array's
 * address (hipGetSymbolAddress) and the launch plan; make it before a
 * capture begins. */
#define BCJR_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
int bcjr_forward_noalloc(const bcjr_problem* prob, const float* seq, const float* T,
                         const float* codebook_or_lut, float* soft, float* logZ,
                         hipStream_t stream);

/* Gradient of sum(g_soft * soft) + sum(g_logZ * logZ) with respect to the
 * sequences, (B, N, V).  g_logZ may be NULL (treated as zero).  logZ is unused
 * (recomputed) and may be NULL.  Codebook and T get no gradient, as in
 * src/bcjr/bcjr_monolithic.py:241-243. */
int bcjr_backward(const bcjr_problem* prob, const float* seq, const float* T,
                  const float* codebook_or_lut, const float* logZ,
                  const float* g_soft, const float* g_logZ, float* g_seq,
                  void* ws, size_t ws_bytes, hipStream_t stream);

/* T -> 0 mode: min-sum Viterbi with the reference's tie rules (lowest
 * predecessor index, lowest final state).  Outputs (any may be NULL):
 *   walk (B, N) int32 states, bitstream (B, N) int32 = walk & (2^kV - 1),
 *   start_state (B,) int32, recon (B, N, V) float32 = c(walk),
 *   mse (B,) float32 mean squared error of recon vs seq,
 *   packed (B, ceil(N*kV/8)) uint8: bitstream packed LSB-first, step t in
 *   bits [t*kV, (t+1)*kV).
 * Replaces viterbi_encode_v_batched_cuda (src/viterbi/cuda_kernel.py:166-220). */
int bcjr_viterbi(const bcjr_problem* prob, const float* seq, const float* codebook_or_lut,
                 int32_t* walk, int32_t* bitstream, int32_t* start_state, float* recon,
                 float* mse, uint8_t* packed, void* ws, size_t ws_bytes, hipStream_t stream);

/* bcjr_viterbi under the tail-biting constraint of viterbi_encode_constrained_v
 * (src/viterbi/encode.py:328-389; V = 1: :105-172): with ob = overlap_bits and
 * v = overlap[b] mod 2^ob, the walk's first state has its top ob bits equal
 * to v and its last state its bottom ob bits equal to v, cost 1e18 standing in
 * for an excluded state as in the reference.  0 <= overlap_bits <= L - k*V
 * (the tail-biting encoder uses L - k*V).  overlap is (B,) int32 on the device.
 * A sequence with no walk meeting the constraint (the reference raises) gets
 * start_state = -1; its other outputs are unspecified. */
int bcjr_viterbi_constrained(const bcjr_problem* prob, const float* seq, const float* codebook_or_lut,
                             int overlap_bits, const int32_t* overlap, int32_t* walk,
                             int32_t* bitstream, int32_t* start_state, float* recon, float* mse,
                             uint8_t* packed, void* ws, size_t ws_bytes, hipStream_t stream);

/* Replay walks: state_t = ((state_{t-1} << kV) | bits_t) & (2^L - 1) from
 * start_state, recon = c(state).  Reads `packed` when non-NULL, else
 * `bitstream`.  walk and recon may be NULL.  Needs no workspace.
 * Replaces viterbi_decode_v (src/viterbi/encode.py:310-325). */
int bcjr_decode(const bcjr_problem* prob, const int32_t* bitstream, const uint8_t* packed,
                const int32_t* start_state, const float* codebook_or_lut, int32_t* walk,
                float* recon, hipStream_t stream);

/* The full min-sum lattice of each sequence: trace[b][t][s] = cum_t(s), the
 * cumulative cost of state s after step t, and backptr[b][t][s] = the
 * predecessor state its minimum chose (the lowest on a tie), with the float32
 * rounding of bcjr_viterbi.  trace (B, N, 2^L) float32, backptr (B, N, 2^L)
 * int32, both caller-owned (2^L * N * 8 bytes per sequence: 128 MiB at L = 16,
 * N = 256).  A diagnostic; needs no workspace.
 * Replaces the return_trace=True outputs of viterbi_encode_v
 * (src/viterbi/encode.py:250-307: trace_err, backpointers). */
int bcjr_viterbi_trace(const bcjr_problem* prob, const float* seq, const float* codebook_or_lut,
                       float* trace, int32_t* backptr, hipStream_t stream);

/* Bitstream layouts accepted by bcjr_dequant. */
enum {
    BCJR_BITS_U8 = 0,     /* (B, N) uint8, one step per byte (the reference's payload) */
    BCJR_BITS_I32 = 1,    /* (B, N) int32, as bcjr_viterbi writes it                   */
    BCJR_BITS_PACKED = 2  /* (B, ceil(N*kV/8)) uint8, kV bits per step, LSB-first      */
};

/* Dequantize an (m, n) matrix of Tx x Ty tiles straight from its bitstreams:
 *   out[r, c] = (float)(scale * c_v(state_t)), the product in double, with
 *   b = (c / Ty) * (m / Tx) + r / Tx,
 *   e = (r % Tx) * Ty + c % Ty = t * V + v,
 * the walk replayed from start_state[b] as in bcjr_decode.  Needs
 * m % Tx == 0, n % Ty == 0, N * V == Tx * Ty and prob->B == (m/Tx) * (n/Ty).
 * The inverse RHT (bcjr_rht with inverse = 1) then gives the weight in the
 * original basis.  Replaces the walk replay + untiling + scaling of
 * dequant_target (src/quantize/serialize.py:56-107) and
 * precompute_walk_states (src/quantize/lut_ft.py:59-79). */
int bcjr_dequant(const bcjr_problem* prob, const void* bitstream, int bits_format,
                 const int32_t* start_state, const float* codebook_or_lut, int64_t m,
                 int64_t n, int Tx, int Ty, double scale, float* out, hipStream_t stream);

/* Materialise the (2^L, V) codebook of prob->code (1MAD, 3INST or HYB; HYB
 * reads the (2^Q, 2) LUT in codebook_or_lut).  Bit-identical to the
 * reference generators. */
int bcjr_codebook(const bcjr_problem* prob, const float* lut, float* codebook_out,
                  hipStream_t stream);

/* Fast Walsh-Hadamard transform of each row of a (rows, n) float32 matrix:
 * out[r, :] = scale * H_n x[r, :] with H_n the unscaled Sylvester Hadamard
 * matrix, butterflies in the order of fwht_numpy (src/rht/transform.py:26-42).
 * n a power of two, 1 <= n <= 16384; out may equal x.  Replaces
 * fast_hadamard_transform.hadamard_transform as called by src/rht/transform.py:44-55
 * and src/qat/ste.py:113-135. */
int bcjr_hadamard(const float* x, float* out, int64_t rows, int64_t n, float scale,
                  hipStream_t stream);

/* Random Hadamard transform of an (m, n) float32 matrix W (m, n powers of two,
 * 1 <= m, n <= 16384), sign vectors sign_l (m) and sign_r (n):
 *   inverse = 0: out = H_m diag(sign_l) W diag(sign_r) H_n / sqrt(m*n)
 *   inverse = 1: out = diag(sign_l) H_m W H_n diag(sign_r) / sqrt(m*n)
 * out must not alias W.  Replaces apply_rht_gpu / apply_inverse_rht_gpu
 * (src/qat/ste.py:113-135) and apply_rht / apply_inverse_rht
 * (src/rht/transform.py:65-126). */
int bcjr_rht(const float* W, float* out, int64_t m, int64_t n, const float* sign_l,
             const float* sign_r, int inverse, hipStream_t stream);

/* bcjr_rht over a batch of (m, n) matrices W (batch, m, n) with one pair of
 * sign vectors per matrix, sign_l (batch, m) and sign_r (batch, n); matrix e of
 * out is bcjr_rht of matrix e of W, in two launches for the whole batch.  No
 * single reference function: it serves the expert-batched dispatch that
 * replaces the per-expert loop of src/qat/qat_moe_layer.py:106-114 (each
 * expert's QuantizedLinear calling apply_rht_gpu, src/qat/ste.py:113-135). */
int bcjr_rht_batched(const float* W, float* out, int64_t batch, int64_t m, int64_t n,
                     const float* sign_l, const float* sign_r, int inverse, hipStream_t stream);

/* Static name of a status code. */
const char* bcjr_strerror(int status);

/* Detail of the calling thread's most recent failure ("" if none). */
const char* bcjr_last_error(void);

/* Library version string. */
const char* bcjr_version(void);

#ifdef __cplusplus
}
#endif

#endif /* BCJR_HIP_H_ */
