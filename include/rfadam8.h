/*
 * rfadam8.h -- C ABI of the MI355X (gfx950) 8-bit AdamW step library
 * (librfadam8.so).
 *
 * The reference (rollfast, pure Python on JAX/Optax) has no native boundary:
 * its hot path is the Python functions cited beside each entry point below,
 * traced by jax.jit.  This ABI is what an XLA FFI custom-call handler (or any
 * other host binding: ctypes, a C++ training loop) calls in their place.
 *
 * Conventions
 *  - Every pointer argument is a device pointer unless documented otherwise;
 *    sizes are element counts.  No torch or XLA types cross the boundary.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *    Calls only enqueue work on that stream; they never synchronise, except
 *    rf_adam8_step (documented below) and plan creation/destruction.
 *  - Functions return RF_OK or an error code; rf_last_error() returns the
 *    calling thread's last message.  Nothing throws across the ABI.
 *  - Updates are in place (JAX donation semantics): params, moment codes,
 *    moment scales and fallback moments are read and overwritten.
 */
#ifndef RFADAM8_H
#define RFADAM8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Exported entry points (the library is built with hidden visibility). */
#define RF_API __attribute__((visibility("default")))

typedef int32_t rf_status;
#define RF_OK 0
#define RF_ERR_INVALID 1     /* bad argument: shape, dtype, size, null pointer */
#define RF_ERR_HIP 2         /* a HIP runtime call failed */
#define RF_ERR_UNSUPPORTED 3 /* valid for the reference, not implemented here */

/* Element types of params, grads, fallback moments and block scales. */
#define RF_F32 0
#define RF_BF16 1
#define RF_F16 2

/* Moment storage of one leaf (adam8.py:605-630 _init_moment_leaf). */
#define RF_MOMENT_QUANTIZED 0 /* uint8 codes [nblocks*block_size] + f32 scales [nblocks] */
#define RF_MOMENT_F32 1       /* fallback_dtype float32 */
#define RF_MOMENT_BF16 2      /* fallback_dtype bfloat16 */
#define RF_MOMENT_F16 3       /* fallback_dtype float16 */

/* Quantizers (adam8.py:113-187 quantize_blocks `quantizer`). */
#define RF_Q_DYNAMIC_SIGNED 0   /* "bitsandbytes.dynamic.signed.8bit.v1", zero code 127 */
#define RF_Q_DYNAMIC_UNSIGNED 1 /* "bitsandbytes.dynamic.unsigned.8bit.v1", zero code 0 */
#define RF_Q_SYMMETRIC_INT8 2   /* "rollfast.symmetric_int8.neg127_pos127.v1", int8 */

/* rf_adam8_hparams.flags */
#define RF_NESTEROV 1u   /* scale_by_adam8(nesterov=True), adam8.py:341-350 */
#define RF_DECAY_WEAK 4u /* weight decay is a Python scalar: wd*p is computed in the
                            param dtype (JAX weak typing); otherwise in f32 */
#define RF_LR 8u         /* chain ends with scale_by_learning_rate (adamw8) */
#define RF_MOMENT_SR 16u /* adamw8(stochastic_rounding=True): moment requantization SR */
#define RF_PARAM_SR 32u  /* apply_updates(stochastic=True) for bf16 params (fused step) */
#define RF_EXACT 128u    /* IEEE div/sqrt in the update direction (bit-exact params);
                            default uses hardware rcp/sqrt (params within 1 bf16 ulp) */
#define RF_FED_BITS 256u /* SR consumes the leaves' *_bits arrays instead of in-kernel
                            Threefry-2x32 */
#define RF_PACKED_BITS 1024u /* no reference counterpart (opt-in): in-kernel SR bits from the
                            packed stream instead of jax.random.bits' one Threefry-2x32-20
                            block per 32-bit word.  Param SR of element e takes the 16-bit
                            half (e & 1) of word (e & 2 ? y1 : y0) of threefry(param key,
                            (hi32(e >> 2), lo32(e >> 2))): a block per four elements.
                            Element e's moment main halves are the 16-bit halves (e & 1)
                            of y0 (first moment) and y1 (second) of threefry(first-moment
                            key, (hi32(e >> 1), lo32(e >> 1))): a block per pair of
                            elements for both; its fill halves are the same halves of the
                            block at counter 2^63 + (e >> 1).  Moment SR draws from the
                            word (main << 16) | fill (its top 23 bits make the uniform;
                            the fill block is computed only for the 2^-16 of draws the
                            main half leaves open); RF_LEAF_STORE_SR rounds with the main
                            half.  Keys are the per-leaf keys of the default stream.
                            Exclusive with RF_FED_BITS */
#define RF_SKIP_NONFINITE 512u /* optax.apply_if_finite reject branch (the wrapper of the
                            fine-tune chain, finetune/builders.py:1605-1609): when any
                            grad of the run is Inf or NaN, the launch leaves the moments
                            untouched and applies a zero update instead (fused step:
                            params become f32(p) + 0 in their dtype, so -0 turns +0;
                            update-only mode: zero updates).  The test reads the grads
                            before clipping. */

/* rf_adam8_leaf.flags */
#define RF_LEAF_DECAY 1u    /* add_decayed_weights applies to this leaf (mask True) */
#define RF_LEAF_SCALE_BF16 8u /* quantized moments: the block scales are stored as bfloat16
                               (scale_dtype, adam8.py:186): computed and used for the codes
                               in f32, stored rounded to nearest even, read back as f32 */
#define RF_LEAF_SCALE_F16 16u /* the same with float16 scales */
#define RF_LEAF_ZERO_DECAY 4u /* optim/adam.py's own decay term with weight 0 (adamw's
                               scale_by_adam gets weight_decay=0.0 and the params,
                               adam.py:185-201, :380-404): the update first becomes
                               u + 0*p in f32 -- NaN for a non-finite param, +0 for a
                               -0 update -- before the RF_LEAF_DECAY term.  Needs the
                               param; unquantized moments only (scale_by_adam8 has no
                               such term) */
#define RF_LEAF_STORE_SR 2u /* bf16 fallback moments are stored with stochastic rounding:
                               bits of split(key_mu | key_nu)[state_index], or mu_bits /
                               nu_bits with RF_FED_BITS (optim/adam.py:219-222 with
                               mu_dtype=bfloat16; adamw8 rounds to nearest even) */

/* One parameter leaf and its optimizer state. */
typedef struct rf_adam8_leaf {
    void* param;        /* [size] param_dtype; read (decay/apply), written by the fused step */
    const void* grad;   /* [size] grad_dtype */
    float* updates;     /* [size] f32 output of the update-only (Optax) mode, else NULL */
    void* mu;           /* quantized: uint8 [nblocks*block_size]; fallback: [size] f32/bf16/f16 */
    float* mu_scales;   /* quantized: [nblocks] block scales, f32 or (RF_LEAF_SCALE_*) 16-bit
                           patterns; fallback: NULL */
    void* nu;           /* as mu (unsigned codebook) */
    float* nu_scales;
    const uint32_t* mu_bits;    /* RF_FED_BITS + RF_MOMENT_SR: [nblocks*block_size] raw bits */
    const uint32_t* nu_bits;
    const uint32_t* param_bits; /* RF_FED_BITS + RF_PARAM_SR: [size] raw bits */
    int64_t size;               /* elements of the leaf (QuantizedBlocks.size) */
    int32_t block_size;         /* QuantizedBlocks.block_size (quantized leaves) */
    int32_t param_dtype;        /* RF_F32 | RF_BF16 | RF_F16 */
    int32_t grad_dtype;         /* RF_F32 | RF_BF16 | RF_F16 */
    int32_t moment_kind;        /* RF_MOMENT_* */
    int32_t state_index;        /* position in the flattened moment template: the per-leaf
                                   moment-SR key is split(key_mu|key_nu)[state_index]
                                   (adam8.py:644-646) */
    int32_t param_index;        /* position in the flattened params: the param-SR key is
                                   split(key_param)[param_index] (utils.py:682) */
    uint32_t flags;             /* RF_LEAF_* */
    int32_t group;              /* index into rf_adam8_hparams.groups when n_groups > 0
                                   (optax.multi_transform label of the leaf), else 0 */
} rf_adam8_leaf;

/* Per-group scalars of a grouped launch: optax.multi_transform over adamw8 /
 * adamw transforms that share b1, b2, eps, eps_root and the step count but
 * not the learning rate, weight decay or keys (the fine-tune builders' groups,
 * finetune/builders.py:1529-1621). */
typedef struct rf_adam8_group {
    float neg_lr;            /* f32(-lr) of the group's learning rate or schedule (RF_LR) */
    float weight_decay;      /* f32(wd) of the group's add_decayed_weights */
    float one_minus_b1;      /* gradient weight of the group's first-moment EMA (adamw8:
                                f32(1.0 - b1); optim/adam.py: 1 - f32(b1)) */
    uint32_t reserved;       /* 0 */
    uint32_t key_mu[2];      /* the group's moment keys, as rf_adam8_hparams.key_mu/key_nu */
    uint32_t key_nu[2];
} rf_adam8_group;

/* Per-step scalars.  The host derives them exactly as the reference does
 * (adam8.py:322-339, optax add_decayed_weights / scale_by_learning_rate). */
typedef struct rf_adam8_hparams {
    float b1, one_minus_b1;  /* f32(b1), f32(1.0 - b1) */
    float b2, one_minus_b2;
    float bc1, bc2;          /* 1 - b1**count_inc, 1 - b2**count_inc (f32) */
    float bc1_next;          /* 1 - b1**(count_inc + 1) (nesterov) */
    float eps, eps_root;
    float weight_decay;      /* f32(wd) */
    float neg_lr;            /* f32(-lr) or -lr(count) of a schedule */
    uint32_t flags;          /* RF_NESTEROV | RF_DECAY_WEAK | RF_LR | ... */
    uint32_t key_mu[2];      /* jax.random key data of key_mu (adam8.py:306); with
                                RF_LEAF_STORE_SR the first-moment storage key */
    uint32_t key_nu[2];
    uint32_t key_param[2];   /* apply_updates key (utils.py:682) */
    float nesterov_one_minus_b1; /* weight of the bias-corrected gradient in the Nesterov
                                    combination: f32(1.0 - b1) computed in double
                                    (adam8.py:341-350, optim/adam.py:146-160).  adamw8
                                    sets it equal to one_minus_b1; optim/adam.py's EMA
                                    weight one_minus_b1 is 1 - f32(b1) in f32
                                    (utils.py:327-335) and differs from it. */
    float clip_max_norm;     /* > 0: the step first scales the grads by
                                min(1, clip_max_norm / (global L2 norm + 1e-6)) with the
                                norm over all the run's leaves (finetune/transforms.py:20-82
                                clip_by_global_norm, fused); 0: no clipping */
    float* clip_out;         /* optional device f32[2] receiving (scale, norm) of the clipping,
                                or NULL */
    int32_t* finite_out;     /* optional device int32 receiving 1 when every grad of the run
                                is finite, else 0 (optax.apply_if_finite's isfinite), or NULL */
    int32_t* finite_host;    /* optional pinned host int32 (hipHostMalloc) receiving the same
                                flag by a copy enqueued right after the pre-pass, before the
                                step; rf_adam8_plan_wait_prepass waits for it, so a host that
                                needs the flag does not wait for the whole step.  NULL: none */
    const rf_adam8_group* groups; /* host array of n_groups: leaf L takes neg_lr, weight_decay,
                                one_minus_b1 and the moment keys from groups[L.group] instead
                                of the fields above; NULL when n_groups == 0.  The library
                                copies it with the leaf table (plan_run_leaves' staging ring),
                                so it may be reused as soon as the call returns. */
    int32_t n_groups;        /* 0: one group (the fields above); else exactly the plan's group
                                count, 1 + the largest leaf.group at plan creation */
    int32_t reserved0;       /* 0 */
    double* magma_sums;      /* optional device f64[3 * n_leaves]: the run also writes, per
                                leaf of the plan's table, the Magma sums of
                                optim/magma.py:98-106 -- sum(g*m'), sum(g*g), sum(m'*m') over
                                the leaf, with g the (clipped) grad and m' the new first
                                moment before storage -- the sums rf_magma_reduce computes in
                                a pass of its own.  Update-only plans whose every leaf has
                                unquantized moments only (RF_ERR_UNSUPPORTED otherwise, and
                                with RF_SKIP_NONFINITE).  NULL: none */
} rf_adam8_hparams;

typedef struct rf_adam8_plan rf_adam8_plan;

/*
 * Build a reusable launch plan over a fixed set of leaves: validates them,
 * uploads the leaf table and its block/chunk work list to device memory
 * once.  apply != 0: fused step (params written, `updates` unused);
 * apply == 0: Optax update-only mode (f32 updates written, params read).
 * Replaces scale_by_adam8.update_fn + adamw8 chain (adam8.py:304-443) and,
 * fused, rollfast.apply_updates (utils.py:648-708).  Synchronises the
 * current device once (table upload).
 */
RF_API rf_status rf_adam8_plan_create(const rf_adam8_leaf* leaves, int32_t n_leaves, int32_t apply,
                               rf_adam8_plan** out_plan);

/* Enqueue one step of the plan on `stream` (one multi-tensor launch) over
 * the pointers given at creation. */
RF_API rf_status rf_adam8_plan_run(const rf_adam8_plan* plan, const rf_adam8_hparams* hp, void* stream);

/* Enqueue one step over new buffers of the same structure (sizes, dtypes,
 * moment kinds, block sizes, key indices and flags must equal the plan's;
 * only pointers may change -- e.g. fresh gradient buffers each step).  The
 * pointer table travels through a ring of pinned staging slots guarded by
 * events: no allocation and no device synchronisation in steady state. */
RF_API rf_status rf_adam8_plan_run_leaves(rf_adam8_plan* plan, const rf_adam8_leaf* leaves, int32_t n_leaves,
                                   const rf_adam8_hparams* hp, void* stream);

/* Wait until the pre-pass (global norm and finite flag) of the plan's latest
 * run with a finite_host has finished and the flag is in finite_host.  The
 * step itself may still be running.  Returns at once when no run asked for it
 * (an empty run never writes finite_host). */
RF_API rf_status rf_adam8_plan_wait_prepass(const rf_adam8_plan* plan);

/* Number of step-kernel launches, leaves and work units of a plan.  A plan
 * with full blocks of bf16 params and grads launches its generic units
 * (partial blocks, small leaves) inside that launch: one launch for such a
 * tree, one more per other (param, grad) dtype pair with full blocks. */
RF_API rf_status rf_adam8_plan_info(const rf_adam8_plan* plan, int64_t* launches, int64_t* leaves,
                             int64_t* units);

/* Diagnostics, no reference counterpart: the memory ceiling of the plan's
 * fused step.  Enqueues, over the plan's full-block (vectorised) work lists
 * with the step's launch shape and lane layout and the pointers given at
 * creation, a kernel that moves exactly the step's bytes -- reads params,
 * grads, both code arrays and both block scales; writes the params, codes
 * and scales back unchanged -- with no arithmetic.  Timing it beside the
 * step gives the bandwidth the step's byte mix reaches in the same memory
 * placement.  `blocks_out` (host, may be NULL) receives the number of
 * 2048-element blocks moved.  Fused plans (apply != 0) only; it must not
 * overlap a step on the same buffers. */
RF_API rf_status rf_adam8_plan_stream_probe(const rf_adam8_plan* plan, void* stream, int64_t* blocks_out);

/* Free a plan (waits for the device to be idle with respect to its tables). */
RF_API rf_status rf_adam8_plan_destroy(rf_adam8_plan* plan);

/* One-shot convenience: create a plan, run it on `stream`, wait for the
 * stream, destroy the plan.  Allocates and synchronises: use plans in loops. */
RF_API rf_status rf_adam8_step(const rf_adam8_leaf* leaves, int32_t n_leaves, int32_t apply,
                        const rf_adam8_hparams* hp, void* stream);

/*
 * rf_adam8_step without allocation.  No counterpart in the reference (whose
 * hot path is Python traced by jax.jit); it is for callers that cannot
 * allocate device memory inside a step: an XLA FFI handler (which must not
 * allocate behind XLA's allocator), tight serving loops and harnesses that
 * forbid hipMalloc.  It cannot be captured into a HIP graph: on a capturing
 * stream it returns RF_ERR_UNSUPPORTED and enqueues nothing.
 *
 * Same arguments and results as rf_adam8_step (fused or update-only, every
 * flag, clipping, the finite flag and groups), except: it does not
 * synchronise the stream at the end (the work is enqueued on it; a
 * finite_host flag is there once the stream has passed the pre-pass), and
 * it refuses magma_sums (RF_ERR_UNSUPPORTED).  Its leaf and group tables,
 * work lists and norm sums live in one device-scope array of
 * RF_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends); a tree
 * whose tables need more fails with RF_ERR_INVALID before any work is
 * enqueued.  The tables take about 184 B per leaf; with clipping or the
 * finite flag add 8 B per 16,384 elements (Llama-7B: 54 KB, 3.35 MB with
 * clipping).  The host copies the tables with one stream-ordered
 * hipMemcpyAsync from pageable memory, so `leaves` may be reused when the
 * call returns.  The call does not wait for work already on the stream:
 * measured on MI355X (ROCm 7.2), it returned in 0.11 ms with 11.7 ms of
 * work ahead of it on the stream (tests/test_zz_no_alloc.py prints the
 * figure), so a host can enqueue steps ahead through it.
 *
 * Every call on one GPU uses that GPU's single array.  Calls are ordered
 * per GPU: each call's stream first waits for the previous call's launches
 * (an event the library records after them, whatever stream they were on),
 * and concurrent calls from several threads enqueue one after another.  The
 * first call of the library on a device uploads the lookup tables with a
 * synchronous copy.
 */
#define RF_NOALLOC_SCRATCH_BYTES (8u << 20)
RF_API rf_status rf_adam8_step_noalloc(const rf_adam8_leaf* leaves, int32_t n_leaves, int32_t apply,
                                       const rf_adam8_hparams* hp, void* stream);

/*
 * adam8.py:113-187 quantize_blocks on a device array x of `size` elements of
 * x_dtype (RF_F32|RF_BF16|RF_F16; taken as f32, jnp.asarray(x, float32)):
 * values [nblocks*block_size] (uint8 codes, or int8 for the symmetric
 * quantizer; padding included), scales [nblocks] of scale_dtype (computed
 * and used for the codes in f32, stored rounded to nearest even:
 * scales.astype(scale_dtype)).  sr != 0 selects stochastic rounding with raw
 * bits `bits` [nblocks*block_size] when non-NULL, else in-kernel
 * Threefry-2x32 bits of key (key0, key1).
 */
RF_API rf_status rf_blockwise_quantize(int32_t quantizer, const void* x, int32_t x_dtype, int64_t size,
                                int32_t block_size, int32_t sr, uint32_t key0, uint32_t key1,
                                const uint32_t* bits, void* values, void* scales, int32_t scale_dtype,
                                void* stream);

/* adam8.py:190-204 dequantize_blocks: values * f32(scales) (scales of
 * scale_dtype), out [size] of out_dtype (RF_F32|RF_BF16|RF_F16, rounded to
 * nearest even). */
RF_API rf_status rf_blockwise_dequantize(int32_t quantizer, const void* values, const void* scales,
                                  int32_t scale_dtype, int64_t size, int32_t block_size, int32_t out_dtype,
                                  void* out, void* stream);

/* utils.py:342-371 _stochastic_round_bf16: out [size] bf16 bit patterns.  Uses
 * `bits` [size] when non-NULL, else in-kernel Threefry-2x32 bits of key. */
RF_API rf_status rf_sr_bf16(const float* x, int64_t size, uint32_t key0, uint32_t key1,
                     const uint32_t* bits, uint16_t* out, void* stream);

/* rf_sr_bf16 with the packed bit source (no reference counterpart; see
 * RF_PACKED_BITS): element e's noise is the 16-bit half (e & 1) of word
 * (e & 2 ? y1 : y0) of threefry(key, (hi32(e >> 2), lo32(e >> 2))). */
RF_API rf_status rf_sr_bf16_packed(const float* x, int64_t size, uint32_t key0, uint32_t key1, uint16_t* out,
                                   void* stream);

/* One leaf of rollfast.apply_updates (utils.py:648-708). */
typedef struct rf_apply_leaf {
    void* param;             /* [size] param_dtype, updated in place */
    const float* updates;    /* [size] f32 */
    const uint32_t* bits;    /* fed SR bits [size] or NULL */
    int64_t size;
    int32_t param_dtype;     /* RF_F32 | RF_BF16 | RF_F16 */
    int32_t param_index;     /* key = split(key)[param_index] */
} rf_apply_leaf;

/* utils.py:648-708 apply_updates over n leaves: bf16 params take
 * f32(p) + u then SR (stochastic != 0) or RNE; f16 params f32(p) + u
 * rounded to nearest even; f32 params take p + u. */
RF_API rf_status rf_apply_updates(const rf_apply_leaf* leaves, int32_t n_leaves, int32_t stochastic,
                           uint32_t key0, uint32_t key1, void* stream);

/* rf_apply_updates with stochastic rounding from the packed bit source (no
 * reference counterpart; see RF_PACKED_BITS): leaf i's key is
 * split(key)[param_index] as in rf_apply_updates; every leaf's bits must be
 * NULL. */
RF_API rf_status rf_apply_updates_packed(const rf_apply_leaf* leaves, int32_t n_leaves, uint32_t key0,
                                         uint32_t key1, void* stream);

/* One leaf of rf_clip_by_global_norm. */
typedef struct rf_clip_leaf {
    const void* grad;   /* [size] dtype */
    void* out;          /* [size] dtype: grad * scale (may equal grad: in place) */
    int64_t size;
    int32_t dtype;      /* RF_F32 | RF_BF16 | RF_F16 */
    int32_t reserved;   /* 0 */
} rf_clip_leaf;

/* finetune/transforms.py:20-82 clip_by_global_norm as a transform: the global
 * L2 norm of all leaves, scale = min(1, max_norm / (norm + 1e-6)), out = grad *
 * scale in the leaf dtype (bf16 leaves: times bf16(scale), one rounding).
 * `stats` (device f32[2] or NULL) receives (scale, norm).  Enqueues on
 * `stream`; its tables and scratch go through the library's per-device
 * staging ring (no allocation once the ring has grown to the tree). */
RF_API rf_status rf_clip_by_global_norm(const rf_clip_leaf* leaves, int32_t n_leaves, float max_norm,
                                        float* stats, void* stream);

/* One leaf of the Magma pass of scale_by_adam(use_magma=True)
 * (optim/adam.py:127-131, :203-217; optim/magma.py:15-132). */
typedef struct rf_magma_leaf {
    const void* grad;   /* [size] grad_dtype: the raw gradient the step receives */
    const void* mu;     /* [size] mu_dtype: the first moment before this step's EMA */
    float* updates;     /* [size] f32: the step's update, scaled in place by rf_magma_scale */
    int64_t size;
    int32_t grad_dtype; /* RF_F32 | RF_BF16 | RF_F16 */
    int32_t mu_dtype;   /* RF_F32 | RF_BF16 | RF_F16 */
    int32_t key_index;  /* the leaf's position among all leaves of the update tree */
    int32_t reserved;   /* 0 */
} rf_magma_leaf;

/* magma.py:98-106 before the step: per leaf i, sums[3i..3i+2] (device f64) =
 * (sum g*m', sum g*g, sum m'*m') with m' = f32(b1*mu) + f32(one_minus_b1*g),
 * the step's new first moment (utils.py:327-335, :437-467).  Enqueue it
 * before the step, which overwrites mu.  Scratch: the staging ring. */
RF_API rf_status rf_magma_reduce(const rf_magma_leaf* leaves, int32_t n_leaves, float b1, float one_minus_b1,
                                 double* sums, void* stream);

/* magma.py:106-124 after the step: per leaf, the f32 cosine of the sums
 * (denominator at least 1e-12, NaN -> 0, clipped to [-1, 1]), the score
 * s = 0.9 * s_prev + 0.1 * sigmoid(cos / tau) written over scores[i] (device
 * f32), the Bernoulli mask m = uniform(split(key, n_keys)[key_index]) < p,
 * and updates = neg_lr * ((m * s) * updates) (neg_lr = 1: no learning-rate
 * scale, optax scale_by_learning_rate otherwise).  With factor_out (device
 * f32[n_leaves], else NULL) the per-leaf factors m * s are written there and
 * the updates are left for rf_magma_apply_updates (updates may then be
 * NULL).  Scratch: the staging ring. */
RF_API rf_status rf_magma_scale(const rf_magma_leaf* leaves, int32_t n_leaves, const double* sums, float* scores,
                                float p, float tau, uint32_t key0, uint32_t key1, int32_t n_keys, float neg_lr,
                                float* factor_out, void* stream);

/* rf_apply_updates with Magma's scaling folded in (no reference
 * counterpart; the fused form of optim/magma.py:120-122, optax
 * scale_by_learning_rate and utils.py:648-708): row i applies
 * neg_lr * (factor[i] * updates) (factor: device f32[n_leaves]). */
RF_API rf_status rf_magma_apply_updates(const rf_apply_leaf* leaves, int32_t n_leaves, const float* factor,
                                        float neg_lr, int32_t stochastic, uint32_t key0, uint32_t key1,
                                        void* stream);

/* One leaf of optax.MultiSteps' gradient accumulator (the fine-tune
 * builders' wrapper, finetune/builders.py:1614-1620; optax is not vendored
 * in the reference). */
typedef struct rf_accum_leaf {
    const void* grad;   /* [size] grad_dtype: this micro-step's gradient (unused by RF_ACC_ZERO) */
    void* acc;          /* [size] acc_dtype: the accumulator, updated in place */
    int64_t size;
    int32_t grad_dtype; /* RF_F32 | RF_BF16 | RF_F16 */
    int32_t acc_dtype;  /* RF_F32 | RF_BF16 | RF_F16 (accumulator_dtype) */
} rf_accum_leaf;

#define RF_ACC_SUM 0  /* use_grad_mean=False: acc = grad + acc */
#define RF_ACC_MEAN 1 /* use_grad_mean=True: acc = acc + (grad - acc) / (n_acc + 1), Welford's running mean */
#define RF_ACC_ZERO 2 /* acc = 0 * acc: the reset after the k-th micro-step ((1 - emit) * acc; a signed
                       zero, NaN where the accumulator held Inf or NaN) */

/* One accumulation over n leaves: per element in the promoted dtype of grad
 * and accumulator (f32, or their common 16-bit type with every operation
 * rounded to nearest even), stored in acc_dtype.  n_acc is the micro-step
 * counter before this step (MultiStepsState.mini_step). */
RF_API rf_status rf_accumulate(const rf_accum_leaf* leaves, int32_t n_leaves, int32_t mode, int32_t n_acc,
                               void* stream);

/* Host-side: the 256 f32 values of a dynamic codebook (adam8.py:461-503). */
RF_API rf_status rf_codebook(int32_t quantizer, float* out256);

/* Host-side: codes that the kernels' table lookup assigns to the normalised
 * values whose f32 bit patterns are first_bits .. first_bits+count-1
 * (diagnostics of the lookup tables; `out` is host memory). */
RF_API rf_status rf_host_table_codes(int32_t quantizer, uint32_t first_bits, int64_t count, uint8_t* out);

/* Host-side: the upper candidate ui = clip(searchsorted_left(cb, n), 0, 255),
 * n clipped to [cb[0], cb[255]] (adam8.py:549-550), that the moment-SR
 * kernels' table lookup computes for the normalised values whose f32 bit
 * patterns are first_bits .. first_bits+count-1 (diagnostics of the tables;
 * `out` is host memory). */
RF_API rf_status rf_host_search_index(int32_t quantizer, uint32_t first_bits, int64_t count, uint16_t* out);

/* Host-side: the 256 neighbour records {cb[li], cb[ui] - cb[li], RN(1 / that
 * gap) or 0, 0} (li = max(ui - 1, 0)) from which the moment-SR kernels form
 * the Bernoulli probability (n - cb[li]) / (cb[ui] - cb[li]) of
 * adam8.py:558-560 (diagnostics of the tables; `out1024` is host memory). */
RF_API rf_status rf_host_sr_records(int32_t quantizer, float* out1024);

/* Library version string. */
RF_API const char* rf_version(void);

/* ABI revision of this header: 2 since rf_blockwise_quantize and
 * rf_blockwise_dequantize take x_dtype / scale_dtype (revision 1 had no
 * dtype arguments).  The shared object's soname carries it
 * (librfadam8.so.2), so a program linked against another revision does not
 * load this library; a dlopen/ctypes binding compares rf_abi_version() with
 * the RF_ABI_VERSION it was written for. */
#define RF_ABI_VERSION 2
RF_API int32_t rf_abi_version(void);

/* Thread-local message of the last failed call ("" if none). */
RF_API const char* rf_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* RFADAM8_H */
