/*
 * selectssm.h — C ABI of the MI355X (gfx950) selective-scan library.
 *
 * The reference (ihh/selectssm) is pure JAX/Flax and has no FFI; each entry
 * point below replaces one reference function on the hot path, named in its
 * comment as file:line (paths relative to the reference's src/selectssm/).
 *
 * Conventions
 *   - Every buffer is device memory owned by the caller.  The library never
 *     allocates, never synchronises and only enqueues work on `stream`
 *     (a hipStream_t passed as void*; NULL means the legacy default stream).
 *   - Tensor layouts are the reference's: u, delta, y, z, dy, du, ddelta: (B,L,D)
 *     row-major (y, dy and z may have a longer row, desc.ld_y / ld_z);
 *     A, dA: (D,N); Bc, Cc, dB, dC: (B,L,N) (rows may be longer, desc.ld_bc); Dskip, dD: (D,).
 *     delta may be (B,L,1) (desc.delta_broadcast=1, selectssm.py:36, 203-210).
 *   - I/O element type is desc.dtype (f32 or bf16).  A, Dskip, dA, dD and the
 *     checkpoints are always f32; the recurrent state and every accumulator
 *     are f32.
 *   - Return 0 on success, a nonzero SSM_ERR_* code otherwise; the message is
 *     available from ssm_last_error() on the calling thread.  Nothing aborts.
 *   - Functions are reentrant.  Calls on different streams do not share state.
 */
#ifndef SELECTSSM_H
#define SELECTSSM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SSM_ABI_VERSION 9

/* error codes */
#define SSM_OK 0
#define SSM_ERR_INVALID 1     /* bad shape, pointer or flag */
#define SSM_ERR_UNSUPPORTED 2 /* valid request this build does not implement */
#define SSM_ERR_HIP 3         /* HIP runtime error (launch failure, ...) */

/* desc.dtype */
#define SSM_F32 0
#define SSM_BF16 1

/* desc.flags */
#define SSM_REVERSE 1u    /* SelectiveSSM(reverse=True): y written at L-1-t (selectssm.py:167-168, 230-231) */
#define SSM_COMPLEMENT 2u /* channel mirrored, D-1-d: with REVERSE the RC map (rcps.py:10-13); alone, a
                             channel-only map (the reference pairs it with REVERSE, selectssm.py:116) */
#define SSM_SKIP 4u       /* y += u*Dskip with u in the scan domain (selectssm.py:238): the output
                             position (p,q) adds u[p,q]*Dskip[q], u read at the output position itself
                             (for a reverse scan the reference's quirk), unless SSM_SKIP_MAP */
#define SSM_GATE 8u       /* y *= silu(z) (BidirectionalMamba, selectssm.py:335-336) */
#define SSM_DELTA_SOFTPLUS 16u /* delta holds the pre-activation: the scan uses softplus(delta)
                                  (selectssm.py:210) and ssm_bwd's ddelta is the gradient with
                                  respect to that pre-activation */
#define SSM_SKIP_MAP 32u        /* the skip's u is read at a map of the scan position instead of
                                   at the output position: the output position of scan step (t,d)
                                   adds u[S(t,d)]*Dskip[column of S(t,d)], S given by the two bits
                                   below.  Conjugating a SelectiveSSM by a flip G (e.g. the RC map
                                   of an RCPS wrapper, rcps.py:61-72) keeps the scan and moves the
                                   output map to G o F and the skip source to F, F the module's own
                                   flip (selectssm.py:167-168) */
#define SSM_SKIP_REVERSE 64u    /* with SSM_SKIP_MAP: S reverses time, t -> L-1-t */
#define SSM_SKIP_COMPLEMENT 128u /* with SSM_SKIP_MAP: S mirrors channels, d -> D-1-d */
#define SSM_ACCUMULATE 256u     /* backward only (ssm_fwd ignores it): ssm_bwd adds the gate's
                                   gradient to dz (which then holds valid data) instead of
                                   writing it; needs SSM_GATE.  In a conv desc, ssm_conv_bwd adds
                                   to dx.  For inputs two calls share: BidirectionalMamba's tied
                                   gate and in_proj blocks (selectssm.py:320-321) get one gradient
                                   buffer, the second call accumulating into it */

typedef struct ssm_desc {
  int64_t batch;          /* B */
  int64_t seqlen;         /* L */
  int64_t dim;            /* D (channels, D_inner) */
  int64_t dstate;         /* N, 1..32 */
  int32_t dtype;          /* SSM_F32 or SSM_BF16 for u, delta, Bc, Cc, z, y, dy, du, ddelta, dB, dC, dz */
  uint32_t flags;         /* SSM_REVERSE | SSM_COMPLEMENT | SSM_SKIP | SSM_GATE | SSM_DELTA_SOFTPLUS
                             | SSM_SKIP_MAP (with SSM_SKIP_REVERSE | SSM_SKIP_COMPLEMENT)
                             | SSM_ACCUMULATE */
  int32_t delta_broadcast;/* 1: delta is (B,L,1) and shared by all channels */
  int32_t segments;       /* time segments per row: 0 = chosen from the shape, else 1..1024
                             (a row's time axis is split into this many segments that run
                             in parallel, joined by their carries; results agree with 1
                             segment up to fp32 rounding) */
  int64_t ld_y;           /* elements between consecutive time rows of y and dy; 0 = dim.
                             With ld_y > dim, y is a column slice of a (B, L, ld_y) array
                             (batch stride L*ld_y), e.g. one half of BidirectionalMamba's
                             concatenated output (selectssm.py:335-336) */
  int64_t ld_z;           /* the same for z, e.g. z read in place from in_proj's output
                             (selectssm.py:319-321); 0 = dim.  dz is always (B,L,D) */
  int64_t ld_bc;          /* elements between consecutive time rows of Bc, Cc, dB and dC; 0 = dstate.
                             With ld_bc >= 2*dstate, Bc and Cc are column slices of one
                             (B, L, ld_bc) array (batch stride L*ld_bc), e.g. read in place from
                             SelectiveSSM's BC projection output (selectssm.py:191-192), and dB,
                             dC are written into the matching slices of one gradient array */
} ssm_desc_t;

/* Version of this ABI (SSM_ABI_VERSION). */
int ssm_abi_version(void);

/* Thread-local text of the last error on this thread ("" if none). */
const char* ssm_last_error(void);

/* Bytes of the forward residual buffer `ckpt`, needed by ssm_bwd: the states
 * entering each block of the scan's time axis and, with SSM_GATE, y before the
 * gate (B*L*D elements of the I/O type), from which ssm_bwd forms dz.  Opaque
 * to callers.  Returns 0 for an invalid desc. */
size_t ssm_ckpt_bytes(const ssm_desc_t* desc);

/* Bytes of scratch `workspace` that ssm_fwd needs (per-segment carries of a
 * time-split scan).  0 when the desc runs as one segment per row (workspace
 * may then be NULL) and for an invalid desc (ssm_last_error() tells which). */
size_t ssm_fwd_workspace_bytes(const ssm_desc_t* desc);

/* Bytes of scratch `workspace` that ssm_bwd needs (partial sums for dB, dC,
 * dA, dD; per-segment adjoint carries).  Returns 0 for an invalid desc. */
size_t ssm_bwd_workspace_bytes(const ssm_desc_t* desc);

/*
 * Forward selective scan.
 * Replaces: ssm_chunked_scan (selectssm.py:37-109), ssm_recursive_scan
 * (ssmrecscan.py:36-77) and the custom-VJP forward ssm_scan_forward
 * (ssmrecscan.py:85-88), plus the scan-adjacent epilogue of
 * SelectiveSSM.__call__ (selectssm.py:230-238) and the gate of
 * BidirectionalMamba (selectssm.py:335-336) when the flags ask for them.
 *   y[b,p,q] = (scan(u,delta,A,Bc,Cc)[b,t,d] + skip) * gate
 * with (p,q) = (t,d) or the reverse / complement map.
 * Dskip is required iff SSM_SKIP, z iff SSM_GATE.  ckpt (ssm_ckpt_bytes) may
 * be NULL for inference; ssm_bwd needs it.  workspace has
 * ssm_fwd_workspace_bytes (NULL allowed when that is 0).
 */
int ssm_fwd(void* stream, const ssm_desc_t* desc,
            const void* u, const void* delta, const float* A,
            const void* Bc, const void* Cc, const float* Dskip, const void* z,
            void* y, float* ckpt, void* workspace);

/*
 * Backward of ssm_fwd for upstream gradient dy (same layout as y).
 * Replaces the custom-VJP backward ssm_scan_backward / _recursive
 * (ssmrecscan.py:111-181); with flags, also the autodiff of the epilogue
 * (selectssm.py:230-238, 335-336).
 * Outputs du, ddelta (B,L,D or B,L,1), dA (D,N), dB, dC (B,L,N); dD (D,)
 * iff SSM_SKIP; dz iff SSM_GATE.  ckpt is the buffer ssm_fwd filled with the
 * same inputs; workspace has ssm_bwd_workspace_bytes.  Deterministic.
 */
int ssm_bwd(void* stream, const ssm_desc_t* desc,
            const void* u, const void* delta, const float* A,
            const void* Bc, const void* Cc, const float* Dskip, const void* z,
            const float* ckpt, const void* dy,
            void* du, void* ddelta, float* dA, void* dB, void* dC,
            float* dD, void* dz, void* workspace);

/* Size of the static device scratch that ssm_bwd_static uses in place of a workspace. */
#define SSM_STATIC_SCRATCH_BYTES (64u << 20)

/*
 * ssm_bwd without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference: it exists for those callers.
 * The workspace is a static device array of SSM_STATIC_SCRATCH_BYTES (64 MiB)
 * that each GPU holds until the process ends; a desc whose
 * ssm_bwd_workspace_bytes exceeds it is rejected with SSM_ERR_INVALID (call
 * ssm_bwd then).  Same results as ssm_bwd, bit for bit.  The stream must
 * belong to the current device.  Calls that overlap on one GPU share the
 * scratch and race: serialise them (one stream, or events).  Allocates
 * nothing (no hipMalloc / hipFree, no allocating library routine).
 */
int ssm_bwd_static(void* stream, const ssm_desc_t* desc,
                   const void* u, const void* delta, const float* A,
                   const void* Bc, const void* Cc, const float* Dskip, const void* z,
                   const float* ckpt, const void* dy,
                   void* du, void* ddelta, float* dA, void* dB, void* dC,
                   float* dD, void* dz);

/* Buffers of one ssm_fwd call (same meaning and requirements). */
typedef struct {
  const void* u; const void* delta; const float* A; const void* B; const void* C;
  const float* D; const void* z; void* y; float* ckpt; void* workspace;
} ssm_fwd_io_t;

/* Buffers of one ssm_bwd call (same meaning and requirements). */
typedef struct {
  const void* u; const void* delta; const float* A; const void* B; const void* C;
  const float* D; const void* z; const float* ckpt; const void* dy;
  void* du; void* ddelta; float* dA; void* dB; void* dC; float* dD; void* dz; void* workspace;
} ssm_bwd_io_t;

/*
 * Two scans, desc[k] with io[k] for k = 0, 1: the same results as ssm_fwd
 * (resp. ssm_bwd) called for each in turn.  Replaces the forward and reverse
 * SSM calls of BidirectionalMamba (selectssm.py:325-326): when both descs
 * have the same shape (batch, seqlen, dim, dstate, dtype, delta_broadcast,
 * segments and SSM_DELTA_SOFTPLUS), the two scans share launches: the
 * time-split aggregate passes always, and ssm_fwd_pair's main pass when the
 * two also need the same kernel variant (both with or both without the
 * epilogue staging of SSM_GATE / reverse SSM_SKIP; u and delta both 16-byte
 * aligned or both not).  ssm_bwd_pair's main passes run one launch per call
 * (a joint one gained nothing).  Each call keeps its own time segments, so the
 * results are bitwise those of the two calls.  The two calls must not share
 * an output or workspace buffer, and must have the same dtype, with one
 * exception in ssm_bwd_pair: when the second call has SSM_ACCUMULATE, both may
 * name one dz buffer, which then receives the first call's dz plus the
 * second's (the two main passes run in call order).
 */
int ssm_fwd_pair(void* stream, const ssm_desc_t* desc, const ssm_fwd_io_t* io);
int ssm_bwd_pair(void* stream, const ssm_desc_t* desc, const ssm_bwd_io_t* io);

/* ------------------------------------------------------------------------
 * Causal depthwise conv1d + activation: the step before the scan
 * (SelectiveSSM.__call__, selectssm.py:167-185).
 *   u[b,t,d] = act( sum_k w[k,d] * x_s[b, t-(K-1)+k, d] ),  x_s[b,t,d] = 0 for t < 0
 * where x_s is x seen in the scan domain: x itself, or with SSM_REVERSE the
 * time-reversed x (x_s[b,t,d] = x[b,L-1-t,d]) and with SSM_COMPLEMENT also the
 * channel-reversed x (x[b,L-1-t,D-1-d]), read through index maps rather than
 * materialised flips (selectssm.py:167-168).  u is written in the scan domain,
 * as the reference's u is; w (K,D) is the Flax kernel (K,1,D) of shift_conv,
 * indexed by scan-domain channel.
 * ------------------------------------------------------------------------ */

/* conv activation (SelectiveSSM.activation, selectssm.py:176-185) */
#define SSM_ACT_NONE 0
#define SSM_ACT_SILU 1
#define SSM_ACT_RELU 2

typedef struct ssm_conv_desc {
  int64_t batch;          /* B */
  int64_t seqlen;         /* L */
  int64_t dim;            /* D */
  int32_t ksize;          /* K (shift_conv_size), 1..8 */
  int32_t dtype;          /* SSM_F32 or SSM_BF16 for x, u, du, dx; w and dw are f32 */
  uint32_t flags;         /* SSM_REVERSE (time) | SSM_COMPLEMENT (channel), either or both;
                             SSM_ACCUMULATE: ssm_conv_bwd adds to dx */
  int32_t activation;     /* SSM_ACT_* */
  int64_t ld_x;           /* elements between consecutive time rows of x; 0 = dim (x may be a
                             column slice of in_proj's output, selectssm.py:319); dx is always
                             (B,L,D) */
} ssm_conv_desc_t;

/* Bytes of scratch `workspace` that ssm_conv_bwd needs (per-tile dw partial
 * sums).  Returns 0 for an invalid desc. */
size_t ssm_conv_bwd_workspace_bytes(const ssm_conv_desc_t* desc);

/*
 * u (B,L,D) = act(conv(x_s, w)) in the scan domain.
 * Replaces: the flip, nn.Conv(feature_group_count=D, padding=[(K-1,0)],
 * use_bias=False) and the activation of SelectiveSSM.__call__
 * (selectssm.py:167-185).
 */
int ssm_conv_fwd(void* stream, const ssm_conv_desc_t* desc, const void* x, const float* w, void* u);

/*
 * Backward of ssm_conv_fwd for upstream gradient du (scan domain, like u):
 * dx (B,L,D, the original domain of x) and dw (K,D).  The pre-activation is
 * recomputed from x and w.  dx may be NULL (not written); dw may be NULL (then
 * workspace may be NULL too).  Deterministic.
 * Replaces: the autodiff of selectssm.py:167-185.
 */
int ssm_conv_bwd(void* stream, const ssm_conv_desc_t* desc, const void* x, const float* w, const void* du,
                 void* dx, float* dw, void* workspace);

#ifdef __cplusplus
}
#endif

#endif /* SELECTSSM_H */
