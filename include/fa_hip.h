/*
 * fa_hip.h -- C ABI of libfa_hip.so, the MI355X (gfx950) flash-attention
 * forward for grouped-query attention, FP16 in and FP16 out, full
 * (non-causal, the reference's only mode) or causal.
 *
 * Layout: q [B, Hq, Nq, 128], k and v [B, Hkv, Nk, 128], o [B, Hq, Nq, 128],
 * all contiguous FP16 in device memory. Output rows are the normalised
 * softmax(q k^T * scale) v with query head h reading key/value head
 * h / (Hq / Hkv). Any Nq, Nk >= 1 with the automatic tile choice (ragged
 * query and key tails are masked); fa_fwd_lse() also returns the per-row
 * log-sum-exp. With fa_problem.causal set, query row i attends only to keys
 * j <= i (top-left, torch's scaled_dot_product_attention(is_causal=True)) or
 * j <= i + Nk - Nq (bottom-right); a row that sees no key gets O = 0 and
 * lse = -inf.
 *
 * Tiles: the attention kernel works on tiles of 256 rows of a row sequence,
 * the Nq query rows of one (b, h), or -- packed, whenever that needs fewer
 * tiles (grouped-query attention with few query rows per head, e.g. decode)
 * -- the Nq * (Hq / Hkv) rows of one (b, KV head) in position-major order
 * (row r is position r / group of query head hkv * group + r % group). A
 * row's result is the same bit for bit either way; packing only lets the
 * heads that share K and V share a tile.
 *
 * V layouts: the 128-key tile comes in two forms with identical results bit
 * for bit. pp_n128_r2 (and the 64-key tiles) read V^T, a key-permuted
 * transposed copy of v that a prep kernel writes into the workspace before
 * the attention kernel runs; pp_n128_r2_vnat reads v where it lies, through
 * gfx950's transposing LDS reads, with no prep pass over v and no V^T in the
 * workspace, and runs its key loop 1.5-12 % slower. The automatic choice
 * takes pp_n128_r2_vnat for at most 2048 query rows per KV head
 * ((Hq / Hkv) * Nq: decode and other short query ranges against long keys),
 * where the prep pass costs more, and pp_n128_r2 otherwise.
 *
 * Conventions (mirroring the reference's two-phase operator binding):
 *   - every entry point returns 0 on success and a nonzero FA_ERR_* code
 *     otherwise; fa_strerror() names the code;
 *   - nothing here allocates device memory or aborts: the caller owns q, k,
 *     v, o and the workspace, and calls on different streams with different
 *     workspaces are independent. The only library state is, per device, a
 *     flag per kernel recording that its dynamic-LDS limit has been raised,
 *     the CU count, and the address of fa_fwd_noalloc()'s static scratch
 *     array (each set on first use);
 *   - fa_fwd() is asynchronous on the given stream (a hipStream_t passed as
 *     void*, NULL for the default stream);
 *   - calls are made with the tensors' device current (hipSetDevice; torch:
 *     `with torch.cuda.device(...)`), since the per-device state above is
 *     looked up for the current device: a stream of another device is
 *     refused with FA_ERR_DEVICE before anything is enqueued.
 *
 * This header needs no HIP or torch headers, so any FFI (ctypes, cgo, JNI)
 * can bind it directly.
 */
#ifndef FA_HIP_H
#define FA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fa_status {
  FA_OK = 0,
  FA_ERR_NULL = 1,          /* a required pointer is NULL */
  FA_ERR_GEOMETRY = 2,      /* non-positive size, Hq % Hkv != 0, or overflowing sizes */
  FA_ERR_DIM = 3,           /* head dimension other than 128 */
  FA_ERR_TAIL = 4,          /* reserved: no longer returned (every tile masks ragged tails) */
  FA_ERR_ALIGN = 5,         /* a tensor pointer is not 16-byte aligned */
  FA_ERR_WORKSPACE = 6,     /* workspace missing or smaller than fa_fwd_workspace_bytes() */
  FA_ERR_ACC = 7,           /* unknown accumulation variant */
  FA_ERR_SCALE = 8,         /* scale not finite and positive */
  FA_ERR_KERNEL = 9,        /* unknown kernel selector */
  FA_ERR_LAUNCH = 10,       /* the HIP runtime rejected a launch */
  FA_ERR_CAPTURE = 11,      /* capture stats buffer too small */
  FA_ERR_CAUSAL = 12,       /* unknown causal mode */
  FA_ERR_TRACE = 13,        /* trace buffer too small */
  FA_ERR_SCRATCH = 14,      /* fa_fwd_noalloc: workspace need above FA_NOALLOC_SCRATCH_BYTES */
  FA_ERR_SPLIT = 15,        /* split count outside 0..1024, or a negative CU count */
  FA_ERR_DEVICE = 16        /* the stream belongs to another device than the current one */
};

enum fa_acc {
  FA_ACC_FP32 = 0,          /* O accumulated in FP32 registers across all keys */
  FA_ACC_FP16 = 1           /* O rounded to FP16 after every 512 keys (the reference's packet) */
};
/* FP16 accumulator: the matrix cores add each 512-key packet's PV products
 * (FP32) to O, and O is rounded to FP16 at the end of every packet and after
 * the last key -- the reference FP16-O kernel's per-packet merge
 * O16 = fp16(alpha O16 + partial). The row max m is exact (no lazy raise).
 * Range: O is accumulated unnormalised, as
 * sum_j 2^(s_j c - m c) v_j over the keys seen so far, with m the running
 * row max, so every weight is <= 1 but the sum is not. Once that sum leaves
 * the FP16 range (|.| > 65504, e.g. a long row of nearly equal scores whose
 * values have a mean of ~1: Nk * |mean v| > 65504) the accumulator becomes
 * +-inf and the row's output is inf or NaN. The reference's FP16-O kernel has
 * the same limit (its O is FP16 as well). FA_ACC_FP32 has no such limit. */

/* Attention mask. The reference runs full attention only (sparse_mode=0 in
 * backends/npu_fa/backend.py:48, is_causal=False in
 * backends/expert_v2/impl.py:714); the causal modes are additions. */
enum fa_causal {
  FA_CAUSAL_NONE = 0,         /* every query row sees every key */
  FA_CAUSAL_TOP_LEFT = 1,     /* row i sees keys j <= i */
  FA_CAUSAL_BOTTOM_RIGHT = 2  /* row i sees keys j <= i + Nk - Nq */
};

typedef struct fa_problem {
  int64_t batch;            /* B */
  int64_t heads_q;          /* Hq */
  int64_t heads_kv;         /* Hkv, divides Hq */
  int64_t seq_q;            /* Nq */
  int64_t seq_k;            /* Nk */
  int64_t dim;              /* D, must be 128 */
  float scale;              /* softmax scale, normally dim ** -0.5 */
  int32_t acc;              /* enum fa_acc */
  int32_t kernel;           /* 0 = automatic tile choice; k >= 1 forces tile configuration k */
  int32_t causal;           /* enum fa_causal (0 = full attention) */
} fa_problem;

/*
 * Bytes of device workspace fa_fwd() needs for problem *p: 256 bytes for the
 * counter the kernel's workgroups take query tiles from, plus, for a tile
 * that reads V^T (see V layouts above), V^T (B * Hkv * Nk' * 256 bytes), and,
 * with a ragged key tail, zero-padded copies to a whole key block of the
 * selected tile (Nk' keys) of k (V^T tiles) or of k and v (pp_n128_r2_vnat),
 * B * Hkv * Nk' * 256 bytes each. pp_n128_r2_vnat without a key tail reads k
 * and v where they lie and needs the 256-byte counter alone. Replaces phase 1 of the
 * reference's operator call,
 * aclnn<Op>GetWorkspaceSize (backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/
 * binding.py:21-24,74-75), whose host tiling sizes the scratch buffer
 * (project/op_host/fa_fa_nk_nz_vector_fp32_v5_sumpack.cpp:52-87).
 */
int fa_fwd_workspace_bytes(const fa_problem* p, uint64_t* bytes);

/*
 * Enqueue one attention forward on `stream`: o = softmax(q k^T * scale) v.
 * Replaces phase 2 of the reference's operator call, aclnn<Op>(workspace,
 * size, executor, stream) (backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/
 * binding.py:25-27,80), and the external reference op it is checked against
 * (backends/npu_fa/backend.py:36-49). The workspace must hold at least
 * fa_fwd_workspace_bytes(p) bytes; its contents on entry do not matter.
 */
int fa_fwd(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
           void* workspace, uint64_t workspace_bytes, void* stream);

/*
 * fa_fwd() that also writes lse [B, Hq, Nq] FP32 (16-byte aligned, or NULL
 * for none): lse[b][h][i] = ln sum_j exp(scale * q_i . k_j), the statistic a
 * backward pass or a merge of key-sharded partial results needs. The
 * reference exports no such output: its kernels keep the running max and sum
 * of each row in workspace (K32/vector_output.h:22-38), which this output
 * exposes in closed form.
 */
int fa_fwd_lse(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
               float* lse, void* workspace, uint64_t workspace_bytes, void* stream);

/*
 * Element strides of dims B, H and N of q, k, v and o (dim D, the 128
 * head dimensions, must be contiguous): a [B, H, N, 128] view of any layout
 * whose rows are 16-byte aligned, e.g. the sequence-major [B, N, H, 128]
 * tensors FlashAttention-style code produces, whose b, h, n strides are
 * N*H*128, 128 and H*128. Every stride is a non-negative multiple of 8 and
 * the n stride is at least 128. The reference accepts contiguous BNSD
 * tensors only (FP32V/binding.py:89-99); this is an addition.
 */
typedef struct fa_strides {
  int64_t q[3], k[3], v[3], o[3];
} fa_strides;

/*
 * fa_fwd_lse() on strided q, k, v and o (lse stays contiguous [B, Hq, Nq],
 * NULL for none). Same workspace as fa_fwd(); FA_ERR_ALIGN for strides that
 * are not multiples of 8, FA_ERR_GEOMETRY for negative strides, row strides
 * below 128 or a key row span of 2^31 bytes or more.
 */
int fa_fwd_strided(const fa_problem* p, const fa_strides* strides, const void* q, const void* k,
                   const void* v, void* o, float* lse, void* workspace, uint64_t workspace_bytes,
                   void* stream);

/*
 * Capture (debug) mode: fa_fwd_lse() that also records the online-softmax
 * statistics of every query row after every key block of the selected tile,
 * the counterpart of the reference's capture flag, which dumps the running
 * max, running sum, rescale factor and block row sum per packet into its
 * stats buffer (binding.py:40-44, K32/vector_output.h:29-36). Layout: FP32
 * stats[4][nblk][B * Hq * Nq] (row index (b * Hq + h) * Nq + i), in order
 *   m      running max after the block, natural-log units (scale * score);
 *   l      running sum after the block, relative to m;
 *   alpha  factor the previous sum and O were rescaled by at the block;
 *   z      the block's own sum of (FP16-rounded) probabilities, relative to m;
 * so m + ln l is the log-sum-exp of every key so far and m + ln z that of
 * the block. fa_fwd_capture_count() gives the float count and the block size
 * (key blocks nblk = ceil(Nk / block_keys)). Meant for small debug inputs.
 */
int fa_fwd_capture_count(const fa_problem* p, uint64_t* count, int32_t* block_keys);
int fa_fwd_capture(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
                   float* lse, float* stats, uint64_t stats_count, void* workspace,
                   uint64_t workspace_bytes, void* stream);

/*
 * Trace mode: fa_fwd() that also writes one record of 8 uint64 words per
 * 256-row query tile of the attention kernel into trace (16-byte aligned, at least
 * fa_fwd_trace_count() words), the counterpart of the reference kernel's
 * per-core trace output, which records each core's id and its start and end
 * system-counter values (K32/panel_kernel.h:222-225,340-342; buffer
 * binding.py:44). Tile w covers rows 256r .. 256r+255 of row sequence s (see
 * Tiles above: S sequences of R rows, S = B*Hq and R = Nq unpacked, S =
 * B*Hkv and R = Nq*Hq/Hkv packed, s = b*Hq + h or b*Hkv + hkv): w = s *
 * ceil(R/256) + r without a mask, and w = (ceil(R/256) - 1 - r) * S + s with
 * a causal mask (longest tiles first). fa_fwd_trace_count() / 8 is the
 * number of tiles. Record of tile w, words 8w .. 8w+7:
 *   0  HW_ID register (bits 0-31) and XCC_ID (bits 32-35) of wave 0 of the
 *      workgroup that ran the tile
 *   1  s_memrealtime when the tile starts (100 MHz reference clock)
 *   2  s_memrealtime after its key loop
 *   3  s_memtime when the tile starts (shader clock cycles)
 *   4  s_memtime after its key loop
 *   5  tile index w
 *   6  key blocks streamed
 *   7  keys per block
 * so the shader clock the tile ran at is (w4 - w3) / (w2 - w1) * 100
 * MHz. The trace kernel is a separate instantiation of the same tile (the
 * production kernels carry no stamps); its O is the production kernel's.
 */
int fa_fwd_trace_count(const fa_problem* p, uint64_t* count);
int fa_fwd_trace(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
                 uint64_t* trace, uint64_t trace_count, void* workspace, uint64_t workspace_bytes,
                 void* stream);

/*
 * Synchronous debug mode: fa_fwd_lse() (lse may be NULL) through a separate
 * instantiation of the same tile that removes the overlap of loads and
 * compute and poisons every buffer the kernels stage through: the workspace
 * (padded K and V) is filled with FP16 NaN before the prep kernel rewrites
 * it, each query tile fills its whole LDS ring (row pads included) with NaN
 * before its first load, and the loads of each phase complete before that
 * phase ends instead of one phase later. A read of staging memory that no
 * load or prep write filled, or a race between the loads and the operand
 * reads, then changes the output (NaN, or a difference from fa_fwd()); a
 * correct build gives fa_fwd()'s output and lse bit for bit. The
 * counterpart of the reference's SYNCHRONOUS build flag, which adds pipe
 * barriers between stages and writes a poison value into layout gaps
 * (cce_fa_nqkq_nz_resident_v13_q768_pool_i4_p128/project/op_kernel/
 * online_softmax.h:10,60-63; cce_fa_nk_nz_vector_fp32_v5_sumpack/project/
 * op_kernel/cce_fp16_reduce.h:33-42). Slower than fa_fwd(): for debugging.
 * Same workspace as fa_fwd().
 */
int fa_fwd_sync(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
                float* lse, void* workspace, uint64_t workspace_bytes, void* stream);

/*
 * Query-row and key granularity fa_fwd() needs for *p: Nq must be a
 * multiple of *rows and Nk of *keys. Every tile masks ragged query and key
 * tails, so both are 1 for any valid selector. Host-side counterpart of the
 * reference binding's alignment check (binding.py:95), which demands
 * Nq % 256 == 0 and Nk % 512 == 0.
 */
int fa_fwd_tile(const fa_problem* p, int32_t* rows, int32_t* keys);

/*
 * Tile configuration (1..fa_kernel_count()) fa_fwd() would launch for *p,
 * with p->kernel == 0 resolved to the automatic choice. Lets a caller name
 * the kernel it timed, as the reference's profiler identifies a backend's
 * device kernel by name (core/profiler.py:14-25).
 */
int fa_fwd_select(const fa_problem* p, int32_t* kernel);

/* Number of selectable tile configurations (valid fa_problem.kernel values are 1..n). */
int fa_kernel_count(void);

/* Static name of tile configuration `kernel` (1..fa_kernel_count()), or NULL. */
const char* fa_kernel_name(int32_t kernel);

/*
 * fa_fwd() without a caller workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * workspace (fa_fwd_workspace_bytes(): the tile counter, V^T for the V^T
 * tiles, padded copies for a ragged key tail) lives in a static device array
 * of FA_NOALLOC_SCRATCH_BYTES per GPU, which the library holds from module
 * load until the process ends; problems whose fa_fwd_workspace_bytes()
 * exceeds it fail with FA_ERR_SCRATCH before any work is enqueued (64 MiB +
 * 64 KiB covers B * Hkv * Nk' = 131072 keys of V^T, e.g. the B=2 N=131072
 * configuration, and every problem pp_n128_r2_vnat runs without a key
 * tail). Nothing is allocated or freed:
 * the first call on a device looks up that device's array address
 * (hipGetSymbolAddress) and keeps it. Every call on one GPU shares that
 * array and each call overwrites what it uses, so calls that overlap on one
 * GPU (different streams, or threads) race and must be serialised by the
 * caller; the array's contents on entry do not matter.
 * Graph capture: the first call of a problem's tile and variant on a device
 * also does host-side set-up (the scratch address, the kernel's dynamic-LDS
 * limit, the CU count), which is not a stream operation; make that first
 * call outside any capture. After it, a call issues kernel launches only
 * (no memset, no allocation) and can be captured in a HIP graph; replays
 * read the inputs in place (GPU-tested).
 */
#define FA_NOALLOC_SCRATCH_BYTES ((64ull << 20) + (64ull << 10))
int fa_fwd_noalloc(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
                   void* stream);

/*
 * Key-split forward: fa_fwd_strided() (strides may be NULL for contiguous
 * tensors; lse may be NULL) that cuts the key range of every 256-row query
 * tile into `splits` near-equal parts of whole key blocks, runs each
 * (tile, part) as its own work item of the attention kernel (a separate
 * instantiation of the same tile), and combines the parts in a second
 * kernel: each part writes its rows' O normalised by the part's own row sum
 * (FP32) and its log-sum-exp lse_s, and the merge forms
 * O = sum_s exp(lse_s - M) O_s / sum_s exp(lse_s - M), M = max_s lse_s,
 * lse = M + ln sum_s exp(lse_s - M). For problems with fewer query tiles
 * than the GPU has CUs (short query ranges, small batch against long keys)
 * this keeps every CU busy; fa_fwd() runs one work item per tile and leaves
 * the rest idle. The results equal fa_fwd_lse()'s up to FP32 summation order
 * (FP16 accumulator: each part rounds its own 512-key packets). splits = 0
 * picks the count automatically on the current device (fa_fwd_split_count),
 * n >= 1 is clamped to the key blocks of the tile, and a count of 1 is
 * exactly fa_fwd_lse(). Workspace: fa_fwd_split_workspace_bytes(), which
 * adds (4 + 512) * splits bytes per query row to fa_fwd_workspace_bytes().
 * The reference has no counterpart: its task split covers (batch * head,
 * query block) only (K32/cce_task.h:28-35); this is the single-GPU form of
 * a key-sharded forward, whose per-shard (O, lse) pairs merge the same way.
 */
int fa_fwd_split_count(const fa_problem* p, int32_t splits, int32_t cus, int32_t* effective);
int fa_fwd_split_workspace_bytes(const fa_problem* p, int32_t splits, uint64_t* bytes);
int fa_fwd_split(const fa_problem* p, int32_t splits, const fa_strides* strides, const void* q,
                 const void* k, const void* v, void* o, float* lse, void* workspace,
                 uint64_t workspace_bytes, void* stream);
/* fa_fwd_split_count: the effective part count for a requested one (0 =
 * automatic) on a GPU with `cus` compute units (0 = the current device's):
 * the automatic choice models the launch's duration per candidate count up
 * to 256 (work items per CU, per-item overhead, the merge's HBM traffic or,
 * with few rows, its walk over the parts; for at most 4096 rows and 32 parts
 * or more the merge gives each row a workgroup) and splits only when that
 * beats one pass over the keys by 10 %. */

/* Static message for a status code. */
const char* fa_strerror(int status);

#ifdef __cplusplus
}
#endif

#endif /* FA_HIP_H */
