/*
 * brx.h -- C-ABI of the MI355X (gfx950) routed-expert MoE library, libbrx.so.
 *
 * The library replaces the per-layer expert arithmetic and the slot pool behind BigRig's
 * `StreamingSwitchGLU` (bigrig_engine/stream.py:814-1631) and `ExpertPool`
 * (bigrig_engine/stream.py:454-811), which the reference runs as MLX ops
 * (`mx.gather_qmm` stream.py:1623-1625, `mx.quantized_matmul` stream.py:1261-1266,
 * the router softmax/argpartition the reference restates at stream.py:895 and 1436-1439).
 *
 * Conventions
 *   - Every entry point returns 0 on success or a negative BRX_E* code; brx_last_error()
 *     returns a message for the last failure on the calling thread. Arguments are validated
 *     before any device memory is written (the reference validates before touching a slot,
 *     stream.py:696-703).
 *   - Device pointers are plain `void*` (from hipMalloc, or torch's data_ptr()); streams are
 *     `hipStream_t` passed as `void*` (NULL = the null stream). Work is stream-ordered.
 *   - bf16 tensors are uint16 bit patterns. Shapes are row-major.
 *   - No entry point is internally thread-safe; use one pool/context per host thread.
 */
#ifndef BRX_H
#define BRX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BRX_ABI_VERSION 2

enum {
    BRX_OK = 0,
    BRX_EINVAL = -1,   /* bad argument: the reference raises ValueError */
    BRX_ESTATE = -2,   /* wrong state (not built, freed): RuntimeError */
    BRX_EHIP = -3,     /* a HIP runtime call failed */
    BRX_ENOMEM = -4,   /* device or pinned allocation failed */
    BRX_ERANGE = -5    /* index out of range (expert id, slot): KeyError */
};

/* quant_mode */
enum { BRX_QUANT_AFFINE = 0, BRX_QUANT_MXFP4 = 1, BRX_QUANT_NONE = 2 };   /* NONE: bf16 weights */
/* scale_dtype (affine only) */
enum { BRX_SCALE_BF16 = 0, BRX_SCALE_F16 = 1 };
/* act: the expert's activation (stream.py:1164-1169) */
enum { BRX_ACT_SWIGLU = 0,          /* silu(gate) * up                                   */
       BRX_ACT_SWIGLU_CLAMPED = 1,  /* gpt-oss: g=min(g,L); u=clip(u,-L,L);
                                         g*sigmoid(alpha*g)*(u+1)                          */
       BRX_ACT_SILU_MLP = 2 };      /* plain two-layer expert (SwitchMLP): fc2(silu(fc1 x)),
                                       projections fc1 [I, H] and fc2 [H, I] packed in that
                                       order (stream.py:57, 1167-1169); layout slot 1 absent */
/* route_mode: the router rule of the MoE block (bigrig_engine/adapter.py:75-93: softmax or
 * sigmoid scoring, optionally group-limited, optionally normalised) */
enum { BRX_ROUTE_SOFTMAX_TOPK = 0,        /* p=softmax(logits); w=p[idx] (OLMoE)           */
       BRX_ROUTE_SOFTMAX_TOPK_RENORM = 1, /* ... then w /= sum(w) (Qwen3 norm_topk_prob)   */
       BRX_ROUTE_TOPK_SOFTMAX = 2,        /* w = softmax(logits[idx]) (gpt-oss)            */
       BRX_ROUTE_SIGMOID_TOPK = 3,        /* s=sigmoid(logits); select on s + bias;
                                             w = s[idx] (DeepSeek-V3-style scoring)        */
       BRX_ROUTE_SIGMOID_TOPK_RENORM = 4 };/* ... then w /= sum(w)                          */
/* router weight dtype */
enum { BRX_DT_F32 = 0, BRX_DT_BF16 = 1 };

/* One MoE layer's shape and quantization: the manifest's per-layer
 * {n_experts, spec, quant} record (stream.py:133-151) plus the block's routing rule. */
typedef struct brx_layer_desc {
    int32_t hidden;        /* H: model width, input of gate/up, output of down (<= 8192)  */
    int32_t inter;         /* I: expert intermediate width (<= 8192)                        */
    int32_t n_experts;     /* E                                                             */
    int32_t top_k;         /* k                                                             */
    int32_t quant_mode;    /* BRX_QUANT_*                                                   */
    int32_t bits;          /* affine: 2, 3, 4, 6 or 8 (codes LSB first); mxfp4: 4; none: 16 */
    int32_t group_size;    /* 64 or 128 (affine), 32 (mxfp4), 0 (none)                      */
    int32_t scale_dtype;   /* BRX_SCALE_* (affine)                                          */
    int32_t has_bias;      /* projections carry a `bias` [N] bf16 component (gpt-oss)       */
    int32_t act;           /* BRX_ACT_*                                                     */
    float   alpha;         /* clamped SwiGLU alpha (1.702)                                  */
    float   limit;         /* clamped SwiGLU limit (7.0)                                    */
    int32_t route_mode;    /* BRX_ROUTE_*                                                   */
    int32_t router_dtype;  /* BRX_DT_*: dtype of the router weight [E, H]                   */
    int32_t shared_inter;  /* intermediate width of an always-on shared expert, 0 = none
                              (any multiple of 64 up to 8192, independent of inter)          */
    /* Group-limited selection (n_group > 1): the experts form n_group contiguous groups of
     * E / n_group; each group is scored (softmax modes: its largest logit; sigmoid modes: the
     * sum of its two largest selection scores s + bias), the topk_group best groups stay
     * eligible (ties to the lower group) and the others drop out of the top-k (sigmoid modes:
     * their selection scores become 0; softmax modes: they are never picked). 0 or 1: none. */
    int32_t n_group;
    int32_t topk_group;
    float   route_scale;   /* routed_scaling_factor: every routing weight is multiplied by it
                              (0 means 1)                                                     */
    int32_t reserved[2];
} brx_layer_desc;

/* Byte offsets of one expert's components inside its packed region, in the order
 * pack_experts writes them (projections gate/up/down -- or fc1/-/fc2 for BRX_ACT_SILU_MLP --
 * components weight/scales/biases/bias, stream.py:152-164). -1 marks an absent component. */
typedef struct brx_expert_layout {
    int64_t weight[3];
    int64_t scales[3];
    int64_t biases[3];
    int64_t bias[3];
    int64_t bytes_per_expert;
} brx_expert_layout;

typedef struct brx_pool brx_pool;

/* ---------------------------------------------------------------- library */
int brx_abi_version(void);
const char* brx_last_error(void);
/* Select the device every later call uses and check it is gfx950. */
int brx_init(int device);

/* Layout of one routed expert (inter = desc->inter) or of the shared expert
 * (shared != 0: inter = desc->shared_inter). Replaces the manifest arithmetic of
 * stream.py:133-141 and ExpertPool.bytes_per_expert (stream.py:539-541). */
int brx_expert_layout_get(const brx_layer_desc* d, int shared, brx_expert_layout* out);

/* ---------------------------------------------------------------- pool
 * C expert slots for ONE layer in HBM plus a device expert->slot table, the residency
 * structure of ExpertPool (stream.py:454-811). The host keeps the authoritative tables and
 * the eviction policy (ExpertPool.touch/_victim/admit, stream.py:622-780); the device only
 * holds bytes and the table kernels read. */

/* Allocate `capacity` slots of bytes_per_expert each (ExpertPool.build, stream.py:570-597).
 * 1 <= capacity <= n_experts (stream.py:503-506). The table starts with every expert absent
 * (-1). */
int brx_pool_create(const brx_layer_desc* d, int capacity, brx_pool** out);
/* Free the slots (StreamHandle.close, stream.py:2160-2191). Synchronizes the pool's streams. */
int brx_pool_destroy(brx_pool* p);
int brx_pool_capacity(const brx_pool* p);
/* Device address of slot `slot` (the expert's bytes, blob layout). */
int brx_pool_slot_ptr(brx_pool* p, int slot, void** out);
/* Device address of the int32 expert->slot table [n_experts] kernels read. The table is
 * read-only for the caller: change it only through brx_pool_set_g2s (or, on a host-backed pool,
 * brx_pool_publish_async / brx_pool_admit_async). The pool's count of resident entries, which
 * brx_moe_block_forward checks before it launches anything, follows those calls only; a table
 * edited through this pointer leaves it stale. */
int brx_pool_g2s_ptr(brx_pool* p, int32_t** out);

/* Copy one expert's packed bytes from pinned host memory into slot `slot`, asynchronously on
 * `copy_stream`. The copy first waits for every forward already issued that reads this pool
 * (write-after-read on the slot), and records an event the next forward waits on
 * (read-after-write). nbytes must equal bytes_per_expert (stream.py:696-703).
 * Replaces the slot write of admit_arrays (stream.py:765-769). */
int brx_pool_refill_async(brx_pool* p, int slot, const void* host_src, size_t nbytes,
                          void* copy_stream);
/* n experts into slots slot0 .. slot0 + n - 1 from pinned host memory, expert i at
 * host_src + i * host_stride (nbytes = bytes_per_expert each), ordered as brx_pool_refill_async.
 * When both sides hold the experts back to back (host_stride = slot stride = nbytes) it is one
 * transfer. The reference reads a layer's experts ahead one by one (StreamHandle.read_ahead,
 * stream.py:2009-2034); a whole layer arriving at once is this call. */
int brx_pool_refill_range_async(brx_pool* p, int slot0, int n, const void* host_src,
                                int64_t host_stride, size_t nbytes, void* copy_stream);
/* Same, from device memory (a staged expert, stream.py:957-961). */
int brx_pool_refill_from_device_async(brx_pool* p, int slot, const void* dev_src, size_t nbytes,
                                      void* copy_stream);
/* Upload the host expert->slot table (int32 [n_experts], -1 = absent; ExpertPool.g2s_device,
 * stream.py:791-797), ordered on `stream` and after any refill. An absent expert stays -1 on
 * the device: a forward that routes to it on a pool without host backing does not compute it
 * from another expert's slot (the reference raises KeyError, stream.py:608-615) -- the rows it
 * touches are written as NaN and the pool records the error, which brx_pool_check reports. */
int brx_pool_set_g2s(brx_pool* p, const int32_t* g2s_host, int n, void* stream);
/* Block until every copy and forward issued against the pool has finished. */
int brx_pool_sync(brx_pool* p);
/* brx_pool_sync, then BRX_ERANGE (naming the expert) if a forward since the last check routed
 * to an expert that was neither in a slot nor host-backed; the error is cleared by the report.
 * The device-side counterpart of ExpertPool.expert_arrays' KeyError (stream.py:608-615) for
 * routing the host never sees. */
int brx_pool_check(brx_pool* p);

/* ---- host-served misses (no per-layer host round trip)
 * The reference keeps a bounded layer off the sync-free path because it must read the routing
 * back to find its misses (stream.py:1440-1450, 1579-1603; autoconfig.py:52-109 for the
 * whole-layer trade it forces). With host backing the kernels
 * detect a miss themselves: a table entry of -1 makes them read that expert's bytes from the
 * layer's pinned host store over the bus instead of from a slot, so every layer can take the
 * sync-free path and the host updates residency behind the forwards, from routing it copies
 * back asynchronously.
 *
 * Give the pool host backing: the layer's routed experts in pinned host memory, expert e at
 * host_base + e * host_stride (host_bytes in all), mapped at the same address on the device
 * (checked). host_stride must equal the pool's slot stride (bytes per expert rounded up to
 * 256) and host_base be 256-byte aligned: a host expert is addressed exactly as a slot. Only on
 * a fresh pool (no refill, table upload or forward yet); every table entry starts at -1; the
 * memory must outlive the pool's last forward. */
int brx_pool_set_host_backing(brx_pool* p, const void* host_base, int64_t host_stride,
                              size_t host_bytes);
/* Set n table entries experts[i] -> slots[i] (slot -1: read from host backing) on `stream`, in
 * stream order; the values are kernel arguments, nothing is read from the host later. Used on
 * the compute stream to retire a victim (-1) before its slot is rewritten. Host backing
 * required; experts distinct. */
int brx_pool_publish_async(brx_pool* p, int n, const int32_t* experts, const int32_t* slots,
                           void* stream);
/* Admit expert `expert` into `slot` behind the forwards: on copy_stream, wait for every forward
 * already issued against the pool, copy the expert's bytes from pinned host memory into the
 * slot, then set table[expert] = slot. Forwards do not wait for it; until the entry lands they
 * read the expert from host backing. The caller retires the slot's previous expert with
 * brx_pool_publish_async(-1) on the compute stream first, and does not retire `expert` again
 * before this copy has finished (the copy stream's table write would land after it). Host
 * backing required. Replaces the slot write of admit_arrays (stream.py:765-769) on this path. */
int brx_pool_admit_async(brx_pool* p, int expert, int slot, const void* host_src, size_t nbytes,
                         void* copy_stream);

/* ---------------------------------------------------------------- compute */

/* Router top-k for T tokens: logits = x . W_r^T (+ bias), then the layer's routing rule.
 *   x        [T, H] bf16 (device)
 *   w_router [E, H] fp32 or bf16 per d->router_dtype (device)
 *   bias     [E] fp32 or NULL: softmax modes add it to the logits (router bias, synthetic
 *            Zipf bias); sigmoid modes add it to the sigmoid scores for selection only (the
 *            score-correction bias), the weights being the uncorrected scores
 *   shared_gate_w [H] bf16 or NULL: shared-expert gate row; out_shared_gate[t] =
 *            sigmoid(x_t . w) when given
 *   out_idx  [T, k] int32: experts by descending logit, ties to the lower id
 *   out_w    [T, k] fp32: routing weights in the same order
 * Logits use one fixed fp32 reduction order so indices are reproducible bit for bit.
 * Replaces the block's gate + softmax + argpartition + take (+ renorm) (stream.py:1436-1439;
 * adapter.py:75-93). */
int brx_router_topk(const brx_layer_desc* d, const void* x, const void* w_router,
                    const float* bias, const void* shared_gate_w, int T,
                    int32_t* out_idx, float* out_w, float* out_shared_gate, void* stream);

/* flags for brx_moe_forward */
#define BRX_FWD_FORCE_DECODE  1u  /* take the gather-GEMV path (at most 8 token rows, 64 pairs;
                                     BRX_EINVAL above)                                       */
#define BRX_FWD_FORCE_PREFILL 2u  /* take the grouped-GEMM path whatever T is              */
/* Split launch: run only the first half (gate/up + act; for the grouped GEMM also the
 * bucketing) or only the second half (down + combine) of a forward. The halves share the
 * library workspace, so a PHASE_B call must follow the PHASE_A call of the same forward with
 * nothing else using the library in between. Both bits or neither = the whole forward. */
#define BRX_FWD_PHASE_A       4u
#define BRX_FWD_PHASE_B       8u
/* brx_moe_block_forward only: the routing step (router logits for T <= 8, the whole router
 * otherwise). Any set of PHASE_R / PHASE_A / PHASE_B runs just those steps, in that order, on
 * the library workspace, under the same rule as PHASE_A / PHASE_B above. */
#define BRX_FWD_PHASE_R      16u

/* The routed experts of one MoE layer for T tokens, reading expert bytes from the pool's
 * slots through its device table (slot = g2s[expert]):
 *   y[t, j]   = down(act(gate(x_t), up(x_t)))  for expert idx[t, j]       (bf16)
 *   out[t]    = sum_j w[t, j] * y[t, j]  (+ shared_gate[t] * shared(x_t)) (fp32 sum, bf16)
 * x [T, H] bf16; idx [T, k] int32; w [T, k] fp32; out [T, H] bf16 or NULL;
 * y_unreduced [T, k, H] bf16 or NULL (the unreduced rows StreamingSwitchGLU returns,
 * stream.py:1377-1577); shared_expert: device pointer to the shared expert's packed bytes
 * (layout brx_expert_layout_get(shared=1)) or NULL; shared_gate [T] fp32 or NULL.
 * Without a FORCE flag, T <= 8 with T * k <= 64 runs the decode gather-GEMV kernels, anything
 * larger the prefill grouped GEMM on MFMA (the reference's per-row `gather_qmm` vs sorted
 * `gather_qmm`, stream.py:1128-1172, 1320-1336). The library keeps a grown-on-demand
 * workspace. An expert in idx that is absent from a pool without host backing yields NaN rows
 * and an error brx_pool_check reports (see brx_pool_set_g2s). */
int brx_moe_forward(const brx_layer_desc* d, brx_pool* p, const void* x, const int32_t* idx,
                    const float* w, const void* shared_expert, const float* shared_gate, int T,
                    void* out, void* y_unreduced, unsigned flags, void* stream);

/* The expert rows of an explicit list of (token, expert) pairs, unreduced:
 *   y_rows[pair_row[i]] = down(act(gate(x[pair_token[i]]), up(x[pair_token[i]])))
 * for expert pair_expert[i], read through the pool's table; expert id n_experts names the
 * shared expert (`shared_expert`, required then). y_rows has n_rows rows; pair_row may be NULL
 * (row i, n_rows >= n_pairs); when given, its entries are distinct rows in [0, n_rows)
 * (entries outside are clamped). This is the span form of the reference's
 * expert-sorted prefill, StreamingSwitchGLU._forward_pairs (stream.py:1320-1336), used when one
 * chunk routes to more experts than the pool holds: the caller cuts the pairs into spans of
 * at most `capacity` experts (_pair_chunks, stream.py:1098-1126), makes each span resident and
 * calls this once per span, writing straight to the unsorted positions (stream.py:1558-1561).
 * x [T, H] bf16. Pass the same FORCE flag for every span of one chunk so a row's arithmetic
 * does not depend on how the chunk was cut (without a flag: decode kernels when n_pairs <= 8
 * and T <= 8, since the decode kernels stage every row of x). */
int brx_moe_forward_pairs(const brx_layer_desc* d, brx_pool* p, const void* x, int T,
                          const int32_t* pair_token, const int32_t* pair_expert,
                          const int32_t* pair_row, int n_pairs, int n_rows,
                          const void* shared_expert, void* y_rows, unsigned flags, void* stream);

/* A whole MoE block for T tokens with every expert resident (the reference's sync-free path,
 * stream.py:1377-1394, where the routing never leaves the device): router top-k as
 * brx_router_topk, the routed experts and the combine as brx_moe_forward, and an always-on
 * shared expert gated by sigmoid(x . shared_gate_w) when shared_gate_w/shared_expert are given
 * (mlx_lm's MoE block around SwitchGLU; stream.py:1523-1525, adapter.py:61-64).
 *   out [T, H] bf16; out_idx [T, k] int32 and out_w [T, k] fp32 optional (device): the routing
 *   the block used, the same values brx_router_topk returns.
 * For T <= 8 with T * k <= 64 (or FORCE_DECODE) the routing is ranked inside the expert kernel,
 * so the block is three launches; anything larger routes first and runs the grouped GEMM. Every
 * expert of the layer must be resident (as last uploaded by brx_pool_set_g2s) unless the pool
 * has host backing: BRX_ESTATE otherwise, before anything is launched. PHASE_R / PHASE_A /
 * PHASE_B split the block into its routing, first-half and second-half launches (timing). */
int brx_moe_block_forward(const brx_layer_desc* d, brx_pool* p, const void* x, const void* w_router,
                          const float* router_bias, const void* shared_gate_w,
                          const void* shared_expert, int T, void* out, int32_t* out_idx,
                          float* out_w, unsigned flags, void* stream);

/* brx_moe_block_forward that allocates nothing. It has no counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments, results and errors; the scratch the
 * call needs (routing logits and weights, the decode entry table and activations, or the
 * prefill bucketing and GEMM intermediates) lives in a library-owned static device array of
 * BRX_NOALLOC_SCRATCH_BYTES per GPU, resolved at brx_init, instead of the grown-on-demand
 * workspace, and no hipMalloc, hipFree or device synchronization is made. A call whose scratch
 * exceeds it fails with BRX_EINVAL before anything is launched (every decode step fits; a
 * Qwen3-30B-shaped prefill chunk fits up to ~350 tokens). Every call on one GPU shares that
 * GPU's array and nothing in it has to start at zero: calls that overlap on one GPU (other
 * streams or host threads) race and must be ordered by the caller. */
#define BRX_NOALLOC_SCRATCH_BYTES (16u << 20)
int brx_moe_block_forward_noalloc(const brx_layer_desc* d, brx_pool* p, const void* x,
                                  const void* w_router, const float* router_bias,
                                  const void* shared_gate_w, const void* shared_expert, int T,
                                  void* out, int32_t* out_idx, float* out_w, unsigned flags,
                                  void* stream);

/* The caller's router-weighted combine of unreduced rows (stream.py:1523-1525):
 *   out[t] = bf16( sum_j w[t, j] * y_routed[t, j]  (+ shared_gate[t] * y_shared[t]) )
 * in fp32, j in order. y_routed [T, k, H] bf16, w [T, k] fp32, y_shared [T, H] bf16 or NULL. */
int brx_combine(const brx_layer_desc* d, const void* y_routed, const float* w, const void* y_shared,
                const float* shared_gate, int T, void* out, void* stream);

/* Test hook: fp32 dequantized weight of projection `proj` (0 gate, 1 up, 2 down) of the
 * expert whose packed bytes start at `expert` (device): out [n_out, n_in] fp32.
 * Replaces mx.dequantize (bigrig_engine/precision.py:186-189). */
int brx_dequant(const brx_layer_desc* d, const void* expert, int proj, int shared, float* out,
                void* stream);

/* Test hook: stable bucketing of T*k (token, expert) pairs by expert, as the reference's
 * np.argsort(pe, kind="stable") (stream.py:1526-1530): out_order [T*k] int32 pair ids sorted
 * by expert, out_offsets [E+1] int32 start of each expert's run. */
int brx_sort_pairs(const brx_layer_desc* d, const int32_t* idx, int T, int32_t* out_order,
                   int32_t* out_offsets, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* BRX_H */
