/*
 * moehip — MI355X (gfx950) kernels for moelab's MoE-layer hot path, as a C ABI.
 *
 * Every pointer argument is device memory owned by the caller (the PyTorch caching allocator,
 * or expert records held by the runtime's caches). No entry point allocates, frees or
 * synchronises: each one enqueues its kernels on `stream` (a hipStream_t; NULL = the null
 * stream) and returns. That keeps every entry point capturable in a HIP graph.
 *
 * Return value: 0 on success, otherwise a MOEHIP_E* code; moehip_last_error() gives the
 * message (thread-local). The Python wrapper turns a non-zero code into RuntimeError, which
 * the moelab runtime already treats as "kernel unavailable, use the fallback"
 * (moelab/runtime.py:346-348, 412-414, 737-741).
 *
 * Record format (moelab/store.py:76-115): one record per expert, fields 64-B aligned inside a
 * 4096-B aligned record. A table row is four int64 device addresses
 * [gate_up.q, gate_up.s, down.q, down.s]; float records repeat [gate_up, gate_up, down, down]
 * (moelab/kernels.py:797, 882); fp8 records follow the int layout with fp32 128x128 block
 * scales. Row weights are fp32 and a weight of 0 means "skip this row" (moelab/kernels.py:322).
 */
#ifndef MOEHIP_H
#define MOEHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOEHIP_ABI_VERSION 4

/* error codes */
#define MOEHIP_OK 0
#define MOEHIP_EINVAL 1       /* bad argument (null pointer, size, unsupported combination) */
#define MOEHIP_ELAUNCH 2      /* the HIP runtime refused the launch */
#define MOEHIP_ENODEV 3       /* no usable gfx950 device */
#define MOEHIP_EIO 4          /* a disk read failed or came back short */

/* record precisions: the `precision` of moelab/store.py:39-45, plus block-scaled fp8 */
#define MOEHIP_PREC_INT4 0
#define MOEHIP_PREC_INT8 1
#define MOEHIP_PREC_F16 2
#define MOEHIP_PREC_BF16 3
#define MOEHIP_PREC_F32 4
#define MOEHIP_PREC_FP8 5

/* activation / output dtypes */
#define MOEHIP_DT_F16 0
#define MOEHIP_DT_BF16 1
#define MOEHIP_DT_F32 2

int moehip_abi_version(void);
/* sizeof(moehip_layer_desc) as compiled into the library (a binding checks its own struct). */
size_t moehip_layer_desc_bytes(void);
const char *moehip_last_error(void);
/* 0 if device `dev` is a gfx950 (MI355X-class) GPU, MOEHIP_ENODEV otherwise. */
int moehip_device_check(int dev);

/*
 * y (O,) = W x for one int4 matrix W = (q (O, I/2) u8, s (O, I/gs) f16), x (I,) in `dtype`,
 * y in `dtype`, fp32 accumulation.
 * Replaces moelab/kernels.py:60-67 `gemv_int4` (Triton `_gemv_int4_kernel`, kernels.py:38-57).
 */
int moehip_gemv_int4(const void *q, const void *s, const void *x, void *y, int O, int I, int gs, int dtype,
                     void *stream);

/*
 * The dense part in int8 (attention projections, shared experts, LM head), one token:
 * y (O,) = W x for W = (q (O, K) int8, s (O, K/gs) fp16 group scales), x (K,) and y in `dtype`,
 * fp32 accumulation. K a multiple of 32, gs a multiple of 16 dividing K; q and x 16-byte aligned.
 * Replaces moelab/denseq.py:32-56 (`_gemv8`, behind `gemv_int8`, denseq.py:59-66).
 */
int moehip_dense_gemv_int8(const void *q, const void *s, const void *x, void *y, int O, int K, int gs, int dtype,
                           void *stream);
/*
 * The multi-token path's weights: w (rows, K) in `dtype` = q * s for rows of the same int8 matrix,
 * the scale rounded to `dtype` first and the product rounded once (as moelab/quant.py:191-205
 * `dequantize(q, s, 8, dtype)` computes it). K a multiple of 16; q 16-byte aligned.
 * Replaces the row-block dequantisation of moelab/denseq.py:95-101 (QLinear.forward, n > 1).
 */
int moehip_dense_dequant_int8(const void *q, const void *s, int rows, int K, int gs, int dtype, void *w, void *stream);

/*
 * Kernel A of the grouped expert FFN: for every table row e < n with w[e] != 0,
 *   h[e, r] = silu(gate_e[r] . x) * (up_e[r] . x),  r < I,
 * where gate_e / up_e are rows r and r+I of the record's gate_up matrix (2I, H), dequantised in
 * registers (int4/int8: (q - 8 | q) * fp16 group scale; fp8: e4m3fn * fp32 block scale).
 * x (H,) in `xdtype`; h (n, I) fp32. If acc_zero is non-null, acc_zero[0:H] is set to 0 in the
 * same launch (the reference's ZERO flag).
 * Replaces moelab/kernels.py:801-815 `_Plan.up` (Triton `_grp4_up` 312-361, `_grp4_up_v4`
 * 494-541, `_grp8_up` 667-709, `_grpf_up` 398-428, `_grp_int4_up` 98-124).
 */
int moehip_grouped_up(int prec, const int64_t *tab, const float *w, const void *x, int xdtype, float *h,
                      float *acc_zero, int n, int I, int H, int gs, void *stream);

/*
 * Kernel B with a deterministic combine:
 *   acc[j] += sum over e = 0..n-1 (table order) with w[e] != 0 of  w[e] * (down_e[j] . h[e]).
 * `partial` is caller-owned scratch of moehip_down_workspace_floats(n, H) floats (any content).
 * Replaces moelab/kernels.py:817-831 `_Plan.down` (Triton `_grp4_down` 363-396 and
 * `_grp4_down_v4` 543-575, `_grp8_down` 711-740, `_grpf_down` 430-451, which add with fp32
 * atomics in a run-dependent order; the order here is fixed, like v1 `_grp_int4_down` 126-148).
 */
int moehip_grouped_down(int prec, const int64_t *tab, const float *w, const float *h, float *acc, int n, int H,
                        int I, int gs, float *partial, void *stream);
size_t moehip_down_workspace_floats(int n, int H);

/*
 * out[t, j] = (accumulate ? out[t, j] : 0) + acc[t, j] (+ add[t, j] if add != NULL), for T rows
 * of H, computed in fp32 and rounded once to `dtype` (out and add share `dtype`).
 * Replaces the graph tail `out.copy_(acc); out.add_(cpu_part)` (moelab/kernels.py:949-950) and
 * `out.add_(acc)` (kernels.py:769, 862, 872, 891).
 */
int moehip_combine(const float *acc, const void *add, void *out, int T, int H, int dtype, int accumulate,
                   void *stream);

/*
 * Router: logits = x W^T rounded to `dtype` (fp32 accumulation), p = softmax(logits) in fp32,
 * top-k with the lowest expert index first among equal logits, optional renormalisation
 * (norm_topk_prob), weights cast to `dtype`.
 * x (T, H) and Wr (E, H) in `dtype`; outputs logits (T, E) `dtype`, idx (T, k) int64,
 * w (T, k) `dtype`, w32 (T, k) fp32 (the weights after the cast, as fp32: what the expert
 * kernels consume, moelab/kernels.py:237). E <= 1024, k <= min(E, 32).
 * Replaces transformers OlmoeTopKRouter.forward (models/olmoe/modeling_olmoe.py:337-346),
 * Qwen3MoeTopKRouter (qwen3_moe:249-267) and Qwen3NextTopKRouter (qwen3_next:757-775), called
 * by moelab at runtime.py:909 and graphs.py:255.
 */
int moehip_router_topk(const void *x, const void *Wr, int T, int H, int E, int k, int renorm, int dtype,
                       void *logits, int64_t *idx, void *w, float *w32, void *stream);

/* HOBBIT policy parameters (moelab/policy.py:50-58); t_mid/t2 < 0 mean "None". */
typedef struct moehip_policy {
    int mode;   /* 0 = hobbit, 1 = hi, 2 = lo, 3 = weight threshold (see t1) */
    float t1;    /* t1_for(layer) + 1e-6 rounded to fp32 (the slack of policy.py:120-122); for mode 3
                  * the threshold itself: level 0 when an expert's routed weight (fp32, as rounded to
                  * the activation dtype) is >= t1, else level 2. Mode 3 has no counterpart in
                  * moelab's policy.py: it is the benchmark configurations' per-expert precision rule
                  * ("fp16 if the gate weight is >= 0.15, else int4"). */
    float t_mid; /* t_mid + 1e-6, or < 0 */
    float t2;    /* t2 + 1e-6, or < 0 */
    int protect; /* 1 if the layer is protected (level 0) */
    int upgrade; /* allow_upgrade: a more precise resident copy may serve the request */
    /* f64 = 1: the one-token rule of moelab's default decode path instead (PrecisionPolicy
     * .levels_one, policy.py:89-98 + 125-137, called by runtime.py:494-517): the weights' total,
     * the running sum of weight / total and the comparisons in float64, against the float64
     * thresholds below (t + 1e-6 as Python computes it; < 0 = None). f64 = 0 is the tensor rule
     * (`levels` / `gpu_levels`, policy.py:110-123, fullgraph.py:101-114) that the T > 1 path and
     * the whole-token graph use. The two differ only when s lies within float32 rounding of a
     * threshold. Batched (T > 1) entry points ignore f64: moelab's T > 1 path is the tensor rule. */
    int f64;
    /* e3 = 1: moelab's cache-miss rule (E3, runtime.py:600-615; policy.py:36-38, `miss_t1`) in the
     * one-token rule (f64 = 1 only): a level-0 slot that no resident copy serves at its level-0
     * precision, with s > miss_t1_64 (= miss_t1 + 1e-6 in float64), is served at level 1. */
    int e3;
    double t1_64;
    double t_mid_64;
    double t2_64;
    double miss_t1_64;
} moehip_policy;

/*
 * Decode-time decision + residency for ONE token (the whole-token-graph path): HOBBIT levels and
 * skip of the k routed experts (policy.py:77-123), level -> precision (lv2p[3],
 * policy.py:188-192), choice of the resident copy (most precise allowed resident precision),
 * and the kernel tables. Inputs: idx (k) int64, w32 (k) fp32, rtab (P, E) int64 device base
 * addresses of this layer's resident records (0 = absent), offs (P, 4) int64 field offsets,
 * planned (P) int32 (1 = a kernel plan exists for that precision).
 * Outputs: tab (P, k, 4) int64 and wtab (P, k) fp32 (rows not chosen get weight 0),
 * info (3, k) fp32 = [expert id, chosen precision or -2 if skipped (-1 = missing), level],
 * miss (1) fp32 += number of non-skipped experts with no usable resident copy.
 * Replaces moelab/fullgraph.py:101-114 `gpu_levels` + 149-171 `FullMoE.layer`, and the host
 * table fill of `GroupedGraph.run` (kernels.py:952-969).
 */
int moehip_decide_table(const int64_t *idx, const float *w32, int k, const moehip_policy *pol, const int *lv2p,
                        const int64_t *rtab, int P, int E, const int64_t *offs, const int *planned, int64_t *tab,
                        float *wtab, float *info, float *miss, void *stream);

/*
 * Token-to-expert dispatch (moelab/runtime.py:471-482, `_decide_general`): pairs (t, j) with
 * skip == 0 (skip may be NULL) are sorted by expert id, stably in pair order t*k+j.
 * Outputs: counts (E) int32, offsets (E+1) int32, sorted_pos (T*k) int32 (pair index t*k+j;
 * entries past offsets[E] are -1), rank (T*k) int32 (position of each pair in the sorted list,
 * -1 if skipped). One workgroup; T*k <= 65536, E <= 1024.
 */
int moehip_dispatch(const int64_t *idx, const uint8_t *skip, int T, int k, int E, int32_t *counts,
                    int32_t *offsets, int32_t *sorted_pos, int32_t *rank, void *stream);

/*
 * Symmetric absmax quantisation of w (O, I) fp32 row-major with one fp16 scale per group of gs
 * columns (moelab/quant.py:104-127 with method="absmax", scales from quant.py:57-61, 74-76),
 * written in the store's packing (quant.py:96-101): bits = 4 -> q (O, I/2) u8, value + 8,
 * low nibble = even column; bits = 8 -> q (O, I) i8. s (O, I/gs) f16. gs even, gs <= 64.
 */
/*
 * The disk tier's record read (moelab/store.py:423-445 ExpertStore.read, 378-401 _read_range,
 * 403-421 _split_reads, 229-255 the direct file): `bytes` bytes at `offset` of the open file into
 * dst (host memory), as `parts` ranges of ceil(bytes / parts) rounded up to 4096 bytes read at
 * once on the library's reader threads. fd is an ordinary descriptor; fd_direct an O_DIRECT one on
 * the same file or -1: a range whose address, offset and length are multiples of 4096 goes through
 * it (no page-cache copy), and falls back to fd if refused (EINVAL, EFAULT). On return
 * *direct_ranges and *fallbacks (either may be NULL) count those ranges. Returns MOEHIP_EIO with
 * the reason on a failed or short read (the reference's "truncated read"). Host only: no HIP
 * call, no device needed.
 */
int moehip_disk_read(int fd, int fd_direct, int64_t offset, void *dst, size_t bytes, int parts, int *direct_ranges,
                     int *fallbacks);

int moehip_quantize(const float *w, int O, int I, int bits, int gs, void *q, void *s, void *stream);

/*
 * The same with the mse scale search (moelab/quant.py:64-93 with method="mse", the int4 store
 * default, moelab/store.py:84-85): per group the fp16 scale of least squared error among
 * (max|w| / qmax) x f and, for int4, (w at the first largest |w|) / -8 x f, f = 1.00, 0.98, ...,
 * 0.70; the first of equal errors wins. Errors are float32 sums in numpy's pairwise order.
 * Scales may be negative (int4). Same sizes and packing as moehip_quantize.
 */
int moehip_quantize_mse(const float *w, int O, int I, int bits, int gs, void *q, void *s, void *stream);

/*
 * GPTQ column sweep of one block (moelab/quant.py:172-186, inside gptq_quantize, quant.py:130-188):
 * rows 0..O-1 of W (float32, row stride ldw), columns i1 .. i1 + nb - 1 (nb <= 128, i1 and nb
 * multiples of gs = 32 or 64), against the block of Hinv (the upper Cholesky factor of H^-1, row
 * stride ldh) at (i1, i1). Left to right: at a group's first column its fp16 scale is chosen from
 * the corrected weights (method 0 absmax, 1 mse), q = rint(w / s) clamped, err = (w - q s) /
 * Hinv[i][i], later columns of the block lose err * Hinv[i][j]. Writes q in the store's packing
 * (int4: byte (i1 + i) / 2 of row stride ldq; int8: byte i1 + i), the block's scales into s (fp16,
 * row stride lds, group (i1 + i) / gs) and the errors into E (float32, row stride lde, column i).
 * W is read only: the caller applies W[:, i1 + nb:] -= E Hinv[i1 : i1 + nb, i1 + nb:] between
 * blocks (a float32 matrix product), as the reference does.
 */
int moehip_gptq_block(const float *W, int ldw, const float *Hinv, int ldh, int O, int i1, int nb, int bits, int gs,
                      int method, void *q, int ldq, void *s, int lds, float *E, int lde, void *stream);

/* Static description of one MoE layer for the fused decode kernel. Precision index p follows
 * the store's order (most precise first, moelab/store.py `precisions`). */
typedef struct moehip_layer_desc {
    int P;              /* number of record precisions (1..4) */
    int E, k, H, I;     /* experts, top-k, d_model, d_ff */
    int dtype;          /* activation dtype (MOEHIP_DT_*) */
    int renorm;         /* norm_topk_prob */
    int prec[4];        /* MOEHIP_PREC_* of precision index p */
    int gs_up[4];       /* group size of gate_up / down for int records */
    int gs_dn[4];
    int planned[4];     /* 1 = kernels run for this precision */
    int lv2p[3];        /* HOBBIT level -> precision index (moelab/policy.py:188-192) */
    int64_t offs[4][4]; /* byte offsets of [gate_up.q, gate_up.s, down.q, down.s] in a record */
    moehip_policy pol;
    /* Qwen3-Next shared expert (transformers Qwen3NextSparseMoeBlock.forward, models/qwen3_next/
     * modeling_qwen3_next.py:786-797): out += sigmoid(x . shared_gate) * FFN_s(x). shared_gate (H)
     * in the activation dtype, NULL = no shared expert; shared_rec[p] = base address of the
     * shared expert's record in precision p (0 = absent; the most precise present copy runs).
     * With a shared expert the workspace is sized for k + 1 rows. */
    const void *shared_gate;
    int64_t shared_rec[4];
} moehip_layer_desc;

/*
 * One MoE layer for ONE decode token in a single launch: router logits (x Wr^T, or the given
 * idx_in / w32_in when Wr is NULL), softmax / top-k / renorm, HOBBIT levels + choice of the
 * resident copy + kernel tables (as moehip_decide_table), kernel-A and kernel-B rows of every
 * chosen record, and out = sum over the table in table order (+ add) (+ out if accumulate), cast
 * to the activation dtype. Optional readouts: logits_out (E), idx_out/w_out/w32_out (k),
 * info (3, k) and miss (+= number of missing experts), as in moehip_router_topk /
 * moehip_decide_table. rtab (P, E) holds the base address of each resident record of this layer.
 * `ws` is caller-owned scratch of moehip_decode_layer_workspace_bytes() bytes, 256-B aligned and
 * zeroed once before its first use; every launch leaves it ready for the next. Launches sharing a
 * workspace must not overlap (one workspace per stream).
 * Kernels: with one record precision and 16-bit activations, on a device whose workgroups are
 * dispatched to XCD b % 8 (checked by moehip_device_check), the XCD-local kernel (routing and the h
 * exchange inside each XCD, one exchange of partial rows between XCDs); otherwise the item kernels.
 * grid: 0 = automatic; > 0 = the item kernels with at most that many workgroups (clamped to what
 * the device holds at once); -1 = the XCD-local kernel when it applies, with its trace format.
 * trace (optional, NULL in production): for the item kernels 3 uint64 per work item = (start, end,
 * workgroup) in the GPU's constant real-time clock, 9 route stamps, then 8 stage stamps per item
 * (tracing adds waits inside the items); for the XCD-local kernel (grid = -1) 16 real-time stamps
 * per workgroup. H, I multiples of 32 and <= 2048, E <= 1024, k <= 32; x and Wr 16-byte aligned;
 * fp32 records are not supported here.
 * Replaces, for decode, the whole moelab/runtime.py:523-770 `run_layer` GPU path when every
 * expert is resident (the A5 whole-token path, moelab/fullgraph.py:149-188 + graphs.py:351-426).
 */
int moehip_decode_layer(const moehip_layer_desc *desc, const void *x, const void *Wr, const int64_t *idx_in,
                        const float *w32_in, const int64_t *rtab, void *out, const void *add, int accumulate,
                        void *logits_out, int64_t *idx_out, void *w_out, float *w32_out, float *info, float *miss,
                        void *ws, size_t ws_bytes, int grid, uint64_t *trace, void *stream);
size_t moehip_decode_layer_workspace_bytes(int P, int k, int E, int H, int I);
/*
 * moehip_decode_layer without a workspace argument and without any allocation: the workspace is a
 * 2 MiB array inside this library, one copy per GPU (found and zero-filled by moehip_device_check,
 * which must have been called for the current device first), with the automatic kernel choice and
 * no trace. No counterpart in the reference: it is for callers that cannot allocate (code under HIP
 * graph capture, serving loops that forbid hipMalloc). A layer whose workspace
 * (moehip_decode_layer_workspace_bytes) exceeds 2 MiB is refused with MOEHIP_EINVAL. All calls on
 * one GPU share its array: calls that overlap on one GPU (two streams at once) race.
 */
int moehip_decode_layer_noalloc(const moehip_layer_desc *desc, const void *x, const void *Wr, const int64_t *idx_in,
                                const float *w32_in, const int64_t *rtab, void *out, const void *add, int accumulate,
                                void *logits_out, int64_t *idx_out, void *w_out, float *w32_out, float *info,
                                float *miss, void *stream);
/*
 * The same layer kernel on explicit table rows, with no routing and no decision: row j of
 * precision p runs record rows_b[p * k + j] (a base address; 0 = unused row) with weight
 * rows_w[p * k + j] (fp32), and out = sum over the rows in table order (+ add) (+ out if
 * accumulate), cast to the activation dtype. desc gives P, prec, group sizes, offs, H, I, dtype
 * and k = rows per precision (E, lv2p, pol, planned are ignored; no shared_gate: a shared expert
 * is one more row). ws: moehip_decode_rows_workspace_bytes(P, k, H, I) bytes, as for
 * moehip_decode_layer. Replaces the kernel sequence of moelab/kernels.py:909-984 (`GroupedGraph`:
 * kernels A and B per precision, then out = acc + cpu_part) in one launch.
 */
int moehip_decode_rows(const moehip_layer_desc *desc, const void *x, const int64_t *rows_b, const float *rows_w,
                       void *out, const void *add, int accumulate, void *ws, size_t ws_bytes, void *stream);
size_t moehip_decode_rows_workspace_bytes(int P, int k, int H, int I);
/* Number of work items (tickets) of one moehip_decode_layer launch for this description, with
 * (with_router = 1) or without the router rows; -1 for a bad description. A grid larger than
 * this is clamped to it; the per-item trace needs 3 * (items + 3) + 8 * items uint64. */
int moehip_decode_layer_work_items(const moehip_layer_desc *desc, int with_router);
/* Copies the workspace's sticky error word (non-zero after a bounded wait expired) to flag_out (device).
 * ws = NULL: the current device's scratch array of moehip_decode_layer_noalloc (MOEHIP_EINVAL before
 * moehip_device_check has set it up); copies only, allocates nothing. */
int moehip_decode_layer_error(const void *ws, void *flag_out, void *stream);

/* Which decode kernel the calling thread's last moehip_decode_layer, moehip_decode_layer_noalloc
 * or moehip_decode_rows call launched (0 before any call). No counterpart in the reference (its
 * Triton kernels have one form each): a host-side readout for tests and benchmarks that must know
 * which of the kernels below produced a result. */
#define MOEHIP_KERNEL_XCD 1        /* k_decode_xcd: one layer per launch, organised by XCD */
#define MOEHIP_KERNEL_XCD_TWO 2    /* k_decode_xcd in two passes (more items than resident workgroups) */
#define MOEHIP_KERNEL_ONE_ITEM 3   /* k_decode_tok: one work item per workgroup */
#define MOEHIP_KERNEL_ITEM_LOOP 4  /* k_decode_layer: a loop over work items */
int moehip_decode_last_kernel(void);
const char *moehip_decode_kernel_name(int kernel);

/*
 * A dependency-free streaming read of a decode layer's bytes in ONE launch: the floor the decode
 * kernels are measured against. Replaces the role of moelab's read floor (profiling.py:81-120,
 * `microbenchmarks`: the expert bytes at the bandwidth a plain streaming product reaches), here at
 * the decode kernel's own grid and bytes. seg_base: HOST array of nseg (<= 32) device addresses of
 * equal segments of seg_bytes (records), then an optional extra segment (the router matrix, NULL
 * with extra_bytes = 0); sizes multiples of 16, segments 16-byte aligned. grid workgroups of 256
 * threads split the bytes evenly (each at most one segment's worth, at most 32 x 4 KB). sink: grid
 * uint32 (device; in practice never written); stamps: NULL or 2 * grid uint64 (device): per
 * workgroup its start and the moment all its words arrived (s_memrealtime, 100 MHz).
 */
int moehip_stream_read(const int64_t *seg_base, int nseg, int64_t seg_bytes, const void *extra, int64_t extra_bytes,
                       int grid, uint32_t *sink, uint64_t *stamps, void *stream);

/*
 * T > 1 tokens (prefill chunks, batched decode) through the experts of one layer, int4 gs64
 * records: the pairs (token, slot) sorted by expert (offsets (E+1), sorted_pos (T*k) = t*k+j,
 * rank (T*k) = position of pair t*k+j in sorted_pos or -1, as written by moehip_dispatch), for
 * each expert e with tab[e] != 0: h = silu(X_e gate^T) * (X_e up^T) and y = w_pair * (h down^T)
 * on MFMA (fp16 operands, exact int4 values, fp32 accumulation and group scales), then
 * out[t] = sum over the token's slots in slot order (+ out if accumulate) (+ add). tab (E, 4)
 * int64 record field addresses (0 row = expert not resident: contributes nothing); x (T, H)
 * and out (T, H) in xdtype (fp16 / bf16); w (T*k) fp32 routing weights. H a multiple of 256, I of 128,
 * gs = 64. ws: moehip_grouped_gemm_workspace_bytes(), 256-B aligned.
 * Replaces moelab/runtime.py:418-436 (`_run_grouped_tokens`, per-expert expert_ffn) and the
 * T > 1 accumulation runtime.py:352-353 (`out.index_add_(0, tok, y * w)`).
 */
int moehip_grouped_gemm(int prec, const int64_t *tab, const void *x, int xdtype, int T, int H, int I, int k, int E,
                        int gs, const int32_t *offsets, const int32_t *sorted_pos, const int32_t *rank, const float *w,
                        void *out, const void *add, int accumulate, void *ws, size_t ws_bytes, void *stream);
size_t moehip_grouped_gemm_workspace_bytes(int T, int k, int H, int I);

/*
 * One MoE layer on a T-token chunk in four launches, int4 gs64 records, 16-bit activations:
 * router logits (as moehip_router_topk), then one launch for the softmax top-k (renorm as given;
 * idx (T*k) int64, w (T*k) in xdtype or null, w32 (T*k) fp32 as moehip_router_topk writes them),
 * the expert buckets and, for bf16, the fp16 copy of x the MFMA tiles read, then the grouped
 * GEMMs and the slot-order combine of moehip_grouped_gemm (out (T, H) in xdtype, + out if
 * accumulate, + add). The pairs' order within an expert depends on scheduling; the output does
 * not (every pair's products and every token's slot-order sum are independent of it). logits
 * (T, E) in xdtype. H a multiple of 512, I of 128, E <= 1024, k <= 32, gs = 64. ws: at least
 * moehip_prefill_layer_workspace_bytes(), 256-B aligned, ZEROED before its first use (the routing
 * counters; every launch leaves them zero).
 * Replaces, for a prefill chunk, the model's gate call (transformers Qwen3MoeTopKRouter /
 * OlmoeTopKRouter.forward, called by moelab at runtime.py:909) followed by
 * moelab/runtime.py:459-492 (expert sort) and :418-436, 352-353 (`_run_grouped_tokens`,
 * `out.index_add_`).
 */
int moehip_prefill_layer(int prec, const int64_t *tab, const void *x, const void *Wr, int xdtype, int T, int H, int I,
                         int k, int E, int gs, int renorm, void *logits, int64_t *idx, void *w, float *w32, void *out,
                         const void *add, int accumulate, void *ws, size_t ws_bytes, void *stream);
size_t moehip_prefill_layer_workspace_bytes(int T, int k, int H, int I, int E);

/*
 * moehip_grouped_gemm over P record tables, one per record precision precs[p] (MOEHIP_PREC_INT4 /
 * INT8 / FP8 / F16 / BF16): tabs (P, E, 4) int64, row (p, e) = the field addresses of expert e's
 * record when the expert runs at precision p (as written by moehip_batch_vote), else 0. Pairs of
 * experts with no non-zero row must carry rank -1 (moehip_batch_vote sets it). precs is a host
 * array. Replaces, for any record precision and mixed precision per expert, moelab/runtime.py:
 * 418-436 (`_run_grouped_tokens`: per expert, expert_ffn on its tokens at the voted precision)
 * and the accumulation runtime.py:352-353.
 */
int moehip_grouped_gemm_multi(int P, const int *precs, const int64_t *tabs, const void *x, int xdtype, int T, int H,
                              int I, int k, int E, int gs, const int32_t *offsets, const int32_t *sorted_pos,
                              const int32_t *rank, const float *w, void *out, const void *add, int accumulate, void *ws,
                              size_t ws_bytes, void *stream);

/*
 * moehip_grouped_gemm_multi with the expert products as batched dequant GEMVs instead of MFMA
 * tiles (for few tokens per expert: batched decode): weight rows streamed whole with 16-byte
 * loads and read once per launch however many tokens the expert has, v_dot2_f32_f16 products
 * against each token's activations; same arguments, workspace and results up to fp32 summation
 * order. items: the work lists written by moehip_batch_decide / moehip_batch_route_decide (P lists
 * of T * k + 1 int32, one per record table), or NULL to build them here. Replaces the same reference code as moehip_grouped_gemm_multi.
 */
int moehip_grouped_gemv_multi(int P, const int *precs, const int64_t *tabs, const void *x, int xdtype, int T, int H,
                              int I, int k, int E, int gs, const int32_t *offsets, const int32_t *sorted_pos,
                              const int32_t *rank, const float *w, void *out, const void *add, int accumulate, void *ws,
                              size_t ws_bytes, const int32_t *items, void *stream);

/*
 * HOBBIT levels of T tokens (moelab/policy.py:110-123 `levels`, the T > 1 branch of
 * runtime.py:459-470): w32 (T, ks) fp32, the first k slots routed; levels (T, ks) int32 and skip
 * (T, ks) uint8 (1 = skipped). Slots k..ks-1 (the shared expert) get level 0 and are never
 * skipped. k <= ks <= 64.
 */
int moehip_batch_levels(const float *w32, int T, int k, int ks, const moehip_policy *pol, int32_t *levels,
                        uint8_t *skip, void *stream);

/*
 * One precision per expert for T > 1 tokens (moelab/runtime.py:484-492 with policy.py:148-154
 * `expert_level`: the most precise level requested by at least hi_vote of the expert's pairs,
 * then level_to_precision through lv2p[3]), the resident copy (as moehip_decide_table: rtab
 * (P, E) device base addresses, 0 = absent; upgrade from pol), and the tables of
 * moehip_grouped_gemm_multi: tabs (P, E + has_shared, 4). Expert E is the shared expert when
 * has_shared (records shared_rec[P], a host array). levels, offsets (E + has_shared + 1) and
 * sorted_pos come from moehip_batch_levels and moehip_dispatch (over E + has_shared experts).
 * An expert with no usable copy gets rank -1 on its pairs and adds their number to miss.
 * info (E + has_shared) fp32 = chosen precision, -1 = missing, -2 = no pairs (may be NULL).
 */
int moehip_batch_vote(const int32_t *levels, int E, int has_shared, const int32_t *offsets, const int32_t *sorted_pos,
                      double hi_vote, const moehip_policy *pol, const int *lv2p, const int64_t *rtab,
                      const int64_t *shared_rec, int P, const int64_t *offs, const int *planned, int64_t *tabs,
                      int32_t *rank, float *info, float *miss, void *stream);

/*
 * moehip_batch_levels + moehip_dispatch + moehip_batch_vote in one launch (one workgroup; the same
 * arguments and results): w32 / idx are (T, ks) with the shared expert (id E) as the last slot
 * when has_shared. T * ks <= 65536, E + has_shared <= 1024. For batched decode, where each of
 * those steps is a few microseconds of launch latency. items (P * (T * ks + 1) int32, or NULL):
 * also the work lists of moehip_grouped_gemv_multi, one per record precision (T <= 256).
 */
int moehip_batch_decide(const float *w32, const int64_t *idx, int T, int k, int ks, const moehip_policy *pol,
                        int32_t *levels, uint8_t *skip, int E, int has_shared, int32_t *counts, int32_t *offsets,
                        int32_t *sorted_pos, int32_t *rank, double hi_vote, const int *lv2p, const int64_t *rtab,
                        const int64_t *shared_rec, int P, const int64_t *offs, const int *planned, int64_t *tabs,
                        float *info, float *miss, int32_t *items, void *stream);

/*
 * The per-token part of moehip_batch_route_decide over many workgroups (two waves per token): softmax
 * top-k of the logits (as moehip_router_topk: idx (T, k) int64, w_out (T, k) in dtype or NULL,
 * w32 (T, k) fp32 holding dtype values) and, when gate != NULL, the shared expert as slot k (as
 * moehip_shared_slot: idx_ext / w_ext (T, k + 1); x (T, H), gate (H) 16-byte aligned). For batches
 * too large for the single-workgroup launch; moehip_batch_decide takes it from there.
 * logits (T, E) fp16 / bf16, E <= 1024, k <= 32.
 */
int moehip_route_tokens(const void *logits, int dtype, int T, int E, int k, int renorm, const void *x,
                        const void *gate, int H, int64_t *idx, void *w_out, float *w32, int64_t *idx_ext, float *w_ext,
                        void *stream);

/*
 * The logits part of moehip_router_topk alone: logits (T, E) = x Wr^T rounded to dtype (the gate's
 * F.linear, transformers modeling_olmoe.py:343), for moehip_batch_route_decide.
 */
int moehip_router_logits(const void *x, const void *Wr, int T, int H, int E, int dtype, void *logits, void *stream);

/*
 * Batched decode from the router logits to the GEMV work list in one launch (one workgroup):
 * softmax top-k per token (as moehip_router_topk: idx (T, k) int64, w_out (T, k) in dtype or NULL,
 * w32 (T, k) fp32 holding dtype values), the shared expert as slot k when gate != NULL (as
 * moehip_shared_slot: idx_ext / w_ext (T, k + 1); x (T, H) and gate (H) 16-byte aligned), then
 * moehip_batch_decide, and the work lists of moehip_grouped_gemv_multi (items, P * (T * ks + 1)
 * int32, or NULL). logits (T, E) fp16 / bf16, E + (gate != NULL) <= 1024, k <= 32.
 */
int moehip_batch_route_decide(const void *logits, int dtype, int T, int E, int k, int renorm, const void *x,
                              const void *gate, int H, int64_t *idx, void *w_out, float *w32, int64_t *idx_ext,
                              float *w_ext, const moehip_policy *pol, int32_t *levels, uint8_t *skip, int32_t *counts,
                              int32_t *offsets, int32_t *sorted_pos, int32_t *rank, double hi_vote, const int *lv2p,
                              const int64_t *rtab, const int64_t *shared_rec, int P, const int64_t *offs,
                              const int *planned, int64_t *tabs, float *info, float *miss, int32_t *items,
                              void *stream);

/*
 * Qwen3-Next shared expert as slot k of every token (transformers Qwen3NextSparseMoeBlock.forward,
 * models/qwen3_next/modeling_qwen3_next.py:786-797): idx_ext (T, k + 1) / w_ext (T, k + 1) =
 * the routed idx (T, k) / w32 (T, k) followed by expert id E with weight sigmoid(x . gate), x .
 * gate and the sigmoid each rounded to the activation dtype. x (T, H), gate (H) in dtype.
 */
int moehip_shared_slot(const void *x, const void *gate, int T, int H, int dtype, const int64_t *idx, const float *w32,
                       int k, int E, int64_t *idx_ext, float *w_ext, void *stream);

/*
 * Checkpoint-style FP8 block quantisation of w (O, I) fp32: per 128 x 128 block
 * scale = amax / 448 (1.0 for an all-zero block), q (O, I) = e4m3fn(w / scale) (round to
 * nearest even, saturating at 448), s (ceil(O/128), ceil(I/128)) fp32 — the
 * `weight_scale_inv` that moelab/quant.py:208-219 multiplies back (fixture rule of moelab
 * tests/conftest.py:52-75). Builds "fp8" records; no counterpart kernel in the reference.
 */
int moehip_quantize_fp8_block(const float *w, int O, int I, void *q, float *s, void *stream);

/*
 * Offload staging (pinned host records -> device record slots) on the copy stream.
 * items[i]: src = pinned host address (hipHostMalloc / torch pin_memory), dst = device record
 * slot, bytes (16-byte multiples, 16-byte aligned). mode MOEHIP_STAGE_KERNEL: one gather kernel
 * for the whole batch that reads the host records directly over the host link (n <= 32; every
 * source must be pinned, which is checked with hipPointerGetAttributes on its first and last
 * byte); MOEHIP_STAGE_SDMA: one hipMemcpyAsync per item. Record the caller's event after it.
 * Replaces moelab/runtime.py:310-326 `_to_fast` (one torch.empty + copy_ per record on
 * copy_stream, runtime.py:186) for the records of a layer's misses or prefetch list
 * (runtime.py:899-951 `_prefetch`).
 */
typedef struct moehip_copy {
    const void *src;
    void *dst;
    uint64_t bytes;
} moehip_copy;
#define MOEHIP_STAGE_KERNEL 0
#define MOEHIP_STAGE_SDMA 1
int moehip_stage_records(const moehip_copy *items, int n, int mode, void *stream);

/*
 * tab[idx[i]] = val[i] for i < n <= 64, as one small kernel on `stream` (host arrays, copied into
 * the launch): tab is a device int64 table of tab_len entries (a layer-major (L, P, E) record
 * table). Enqueued on the copy stream after moehip_stage_records, an entry turns non-zero only
 * once its record has landed; enqueued on the compute stream, a removal is ordered after the
 * kernels that still read the old record. Replaces moelab/fullgraph.py:73-98
 * (`DeviceTable.added/removed/upload`: host table edits + a whole-table H2D copy).
 */
int moehip_table_set(int64_t *tab, int64_t tab_len, const int64_t *idx, const int64_t *val, int n, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MOEHIP_H */
