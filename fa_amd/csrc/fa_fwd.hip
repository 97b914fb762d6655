// Flash-attention forward for MI355X (gfx950): GQA, D = 128, FP16 in/out,
// FP32- or FP16-accumulated O, full (non-causal) or causal attention.
//
// Work decomposition (reference: task = (batch*head, query block), KV head
// = head / group, backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/project/
// op_kernel/panel_kernel.h:264-274): a query tile is BM = 256 query rows of
// one (batch, head), 8 waves x 32 rows. The attention kernel is persistent:
// one workgroup per CU takes tiles from a counter until none are left. For a
// tile it streams the whole key range in blocks of BN keys; each K block and
// V block is staged once in LDS (a ring of slots) and read by every wave,
// and every wave keeps its Q fragments, O accumulators and softmax
// statistics in registers for the whole key loop. Ragged query and key tails
// are masked, the per-row log-sum-exp is written on request, and an optional
// causal mask makes a tile stream only the key blocks up to its diagonal.
// Separate instantiations add the capture (per-block softmax statistics),
// trace (per-tile clock stamps) and synchronous debug modes, and the
// key-split mode: work items are (tile, part of its key range), whose
// partial results a merge kernel combines through their log-sum-exp.
//
// Matrix products run transposed so the softmax is lane-local:
//   S^T = K Q^T   v_mfma_f32_32x32x16_f16, A = K rows from LDS, B = Q^T
//                 from registers. Lane l holds query row l%32 and 16 keys
//                 per 32x32 tile.
//   O^T += V^T P^T  A = V^T from LDS, B = P^T straight from the S^T
//                 registers (converted to FP16). Lane l keeps query row l%32
//                 for all its O registers, so rescaling by alpha is per lane.
// The 32x32 output layout gives a lane keys {8g+4h .. 8g+4h+3} (g = 0..3,
// h = lane/32); the PV step over keys 16s..16s+15 therefore wants, in its k
// slots 8h..8h+7 of dim d = lane%32, keys {16s+4h..+3, 16s+8+4h..+3}: two
// runs of 4 consecutive keys down one column of V. Two ways to feed it:
//   * V^T tiles: a prep kernel writes V^T with exactly that key order inside
//     every 16-key group, so each A fragment is one 16-byte LDS read;
//   * the natural-V tile: V is staged in LDS as it lies in memory ([key][dim]
//     rows, like K), and each A fragment is two transposing LDS reads
//     (ds_read_b64_tr_b16, gfx950), each giving every lane 4 keys of its dim.
// The second needs no pass over V before the attention kernel and no V^T
// workspace, at the price of twice the V operand read instructions (about
// 1.5 % of the key loop); the automatic tile choice takes it where that
// pass is the larger cost (few query rows per KV head).
//
// Online softmax in base 2 with the scale folded in (c = scale*log2(e)):
//   m' = max(m, rowmax(S)),  alpha = 2^((m - m') c),  P = 2^(S c - m' c),
//   l' = alpha l + rowsum(P16),  O' = alpha O + P16 V
// where P16 is P rounded to FP16 (the MFMA operand). The row sum is taken
// over the same rounded values, so numerator and denominator use identical
// weights.
// Semantics follow the reference's FP32 vector softmax
// (project/op_kernel/online_softmax.h:86-224, vector_output.h:22-86 of the
// FP32 variant) and, for FA_ACC_FP16, its FP16-O merge (vector_output.h:
// 130-210 of backends/cce_fa_nqkq_nz_resident_v13_q768_pool_i4_p128).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "../../include/fa_hip.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int HD = 128;               // head dimension
constexpr int PAD_GROUP = 64;         // keys per prep-kernel workgroup
constexpr float NEG_BIG = -1.0e30f;   // finite "minus infinity" for the running max
// Added to the score of a masked key: far below any real score
// (|scale * q.k| <= 128 * 65504^2 ~ 5.5e11) and below NEG_BIG, so the key
// gets P = 0 and can neither raise the running max nor start it.
constexpr float MASKED = -1.0e38f;
constexpr double LOG2E = 1.4426950408889634;
constexpr float LN2 = 0.6931471805599453f;

// Kernel instantiation modes. Capture records the online-softmax statistics
// of every row after every key block; trace records, per query tile, where it
// ran and two clock stamps around its key loop. Sync is the synchronous
// debug mode: every tile's LDS ring starts poisoned with FP16 NaN and each
// phase's loads complete before the phase ends, so a read of LDS no load has
// filled, or a race between the loads and the operand reads, changes the
// output. Split is the key-split mode: a work item is one query tile and one
// of `splits` contiguous parts of its key range, and it writes that part's
// normalised FP32 O and log-sum-exp for a merge kernel to combine. All four
// are separate kernels.
enum KernelMode { MODE_RUN = 0, MODE_CAPTURE = 1, MODE_TRACE = 2, MODE_SYNC = 3, MODE_SPLIT = 4 };
constexpr int kModes = 5;
// FP16 quiet NaN in both halves of a 32-bit word: the poison of sync mode.
constexpr uint32_t NAN16X2 = 0x7e007e00u;

// Trace record of one query tile (64-bit words, record index = tile index):
//   0  hardware placement of the workgroup that ran it: HW_ID register (wave
//      slot, SIMD, CU, shader array, shader engine) in bits 0-31, XCC_ID (the
//      accelerator die, one of 8) in bits 32-35, both read by wave 0
//   1  s_memrealtime when the tile starts (constant 100 MHz reference clock)
//   2  s_memrealtime after its key loop (every wave past the final barrier)
//   3  s_memtime when the tile starts (shader-clock cycles)
//   4  s_memtime after its key loop
//   5  tile index
//   6  key blocks the tile streamed
//   7  keys per block
// The shader clock the tile ran at is (w4 - w3) / (w2 - w1) * 100 MHz.
constexpr int TRACE_WORDS = 8;

// Kernel arguments. v is the V buffer the kernel reads: the prep kernel's
// V^T (contiguous, 128 rows of seq_k keys per KV head) or, for the tile that
// reads V in its natural layout, the caller's v or its padded copy. seq_k is
// the key length of the K and V buffers the
// kernel reads (a multiple of its key block); keys at or past nk_valid are
// zero padding and masked out of the softmax. lse (FP32 [B, Hq, Nq],
// natural-log log-sum-exp of the scaled scores) may be null. stats, when not
// null, receives the online-softmax statistics of every row after every key
// block (capture mode): FP32 [4][seq_k / BN][B * Hq * Nq]
// holding the running max m (natural-log units, scale * score), the running
// sum l relative to m, the rescale factor alpha applied at that block, and
// the block's own row sum z relative to m. trace, in trace mode, receives
// one record of TRACE_WORDS 64-bit words per query tile (see trace_record). c is the softmax scale times
// log2(e). With causal set, query row i sees keys j <= i + causal_off only
// (causal_off = 0 aligns the mask top-left, Nk - Nq bottom-right); a row that
// sees no key gets O = 0 and lse = -inf. qs, ks, vs and os are the element
// strides of q, of the K and natural-layout V buffers read (the caller's k
// and v, or their padded contiguous copies) and of o. In split mode (splits >= 2) the kernel writes,
// instead of o and lse, each part's O normalised by its own row sum into
// opart (FP32 [splits][B * Hq * Nq][128]) and the part's natural-log
// log-sum-exp into lpart (FP32 [splits][B * Hq * Nq]; -inf for a part in
// which the row sees no key, whose opart row then holds zeros).
struct Strides {
  int64_t b, h, n;   // batch, head and row strides in elements; the 128 dims are contiguous
};
struct FaArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  _Float16* o;
  float* lse;
  float* stats;
  uint64_t* trace;
  int* next_tile;      // work-queue counter (workspace), zeroed by the prep kernel
  int tiles;           // query tiles of the launch: B * Hq * ceil(Nq / 256)
  int heads_q, group, seq_q, seq_k, nk_valid;
  int causal, causal_off;
  float c;
  Strides qs, ks, os;
  // Split mode only (after the others, so their argument offsets do not move).
  float* opart;
  float* lpart;
  int splits;          // key-range parts per tile
  Strides vs;
};

// Row n of head h of batch b of a strided [B, H, N, 128] tensor.
template <typename T>
__device__ __forceinline__ T* row_at(T* base, const Strides& st, int b, int h, int n) {
  return base + (int64_t)b * st.b + (int64_t)h * st.h + (int64_t)n * st.n;
}

// Maximum of two scores. IEEE-754 maximum (NaN-propagating) lowers to a
// single v_maximum3_f32 with no operand canonicalization; scores are finite.
__device__ __forceinline__ float smax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Combine a per-lane value with the lane 32 apart (same query row, other
// half of the keys).
__device__ __forceinline__ float half_max(float x) {
  auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return smax(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float half_sum(float x) {
  auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// acc + the FP16 value in half HI (0 = low, 1 = high) of x, one rounding:
// v_fma_mix_f32 with the FP16 operand converted exactly and multiplied by
// 1.0. It runs on the plain VALU pipe; the FP16 dot product v_dot2c_f32_f16
// (one instruction per pair) measured 3-4 % slower as the softmax's row sum,
// beside the matrix products of the other wave on the SIMD.
template <int HI>
__device__ __forceinline__ float add_f16(float acc, h2 x) {
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(x));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(x));
  return acc;
}

__device__ __forceinline__ f32x16 mfma32(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Key slot -> key inside a 16-key group of the transposed V (see header).
__device__ __forceinline__ int vt_key_of_slot(int slot) {
  const int h = slot >> 3, e = slot & 7;
  return (e < 4) ? (4 * h + e) : (8 + 4 * h + (e - 4));
}

// Prep for the tiles that read V transposed: vt[kv][d][key0 + slot] =
// v[kv][key0 + key(slot)][d], one 64-key group per workgroup; keys at or past
// nk_valid become zeros. With kpad non-null the group's K rows are also
// copied to kpad[kv][key0 + r] (zero rows past nk_valid), the padded K a
// masked key tail reads. Grid (nk_pad / 64, B * Hkv), 256 threads; v and k
// hold nk_valid keys per head with strides vs and ks, vt and kpad are
// contiguous with nk_pad keys per head. It also resets the attention
// kernel's tile counter.
__global__ void __launch_bounds__(256) fa_prep_kernel(const _Float16* __restrict__ k,
                                                      const _Float16* __restrict__ v,
                                                      _Float16* __restrict__ vt,
                                                      _Float16* __restrict__ kpad, int nk_valid,
                                                      int nk_pad, int heads_kv, Strides ks,
                                                      Strides vs, int* __restrict__ next_tile) {
  __shared__ _Float16 tile[PAD_GROUP][HD + 8];
  const int tid = threadIdx.x;
  if (blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) *next_tile = 0;   // the attention kernel's work queue
  const size_t kv = blockIdx.y;
  const int b = (int)(kv / heads_kv), hk = (int)(kv % heads_kv);
  const int key0 = blockIdx.x * PAD_GROUP;
  _Float16* kdst = kpad ? kpad + (kv * nk_pad + key0) * HD : nullptr;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid + 256 * j;
    const int r = i >> 4, ch = i & 15;
    const bool valid = key0 + r < nk_valid;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(&tile[r][ch * 8]) =
        valid ? *reinterpret_cast<const u32x4*>(row_at(v, vs, b, hk, key0 + r) + ch * 8) : zero;
    if (kdst)
      *reinterpret_cast<u32x4*>(kdst + (size_t)r * HD + ch * 8) =
          valid ? *reinterpret_cast<const u32x4*>(row_at(k, ks, b, hk, key0 + r) + ch * 8) : zero;
  }
  __syncthreads();
  _Float16* dst = vt + kv * HD * (size_t)nk_pad + key0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid + 256 * j;
    const int d = i >> 3, ch = i & 7;
    h8 val;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int slot = (ch & 1) * 8 + e;
      val[e] = tile[16 * (ch >> 1) + vt_key_of_slot(slot)][d];
    }
    *reinterpret_cast<h8*>(dst + (size_t)d * nk_pad + ch * 8) = val;
  }
}

// Prep for the tile that reads V in its natural layout: resets the attention
// kernel's tile counter and, for a ragged key tail (kpad non-null), writes
// zero-padded copies of K and V: kpad[kv][key] and vpad[kv][key] hold the
// caller's rows for keys below nk_valid and zeros up to nk_pad, one 64-key
// group per workgroup (grid (nk_pad / 64, B * Hkv), 256 threads; k and v hold
// nk_valid keys per head with strides ks and vs, the copies are contiguous).
// Without a tail the attention kernel reads the caller's k and v themselves,
// and this kernel runs as one workgroup.
__global__ void __launch_bounds__(256) fa_pad_kernel(const _Float16* __restrict__ k,
                                                     const _Float16* __restrict__ v,
                                                     _Float16* __restrict__ kpad,
                                                     _Float16* __restrict__ vpad, int nk_valid,
                                                     int nk_pad, int heads_kv, Strides ks,
                                                     Strides vs, int* __restrict__ next_tile) {
  const int tid = threadIdx.x;
  if (blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) *next_tile = 0;   // the attention kernel's work queue
  if (!kpad) return;
  const size_t kv = blockIdx.y;
  const int b = (int)(kv / heads_kv), hk = (int)(kv % heads_kv);
  const int key0 = blockIdx.x * PAD_GROUP;
  _Float16* kdst = kpad + (kv * nk_pad + key0) * HD;
  _Float16* vdst = vpad + (kv * nk_pad + key0) * HD;
  const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid + 256 * j;
    const int r = i >> 4, ch = i & 15;
    const bool valid = key0 + r < nk_valid;
    *reinterpret_cast<u32x4*>(kdst + (size_t)r * HD + ch * 8) =
        valid ? *reinterpret_cast<const u32x4*>(row_at(k, ks, b, hk, key0 + r) + ch * 8) : zero;
    *reinterpret_cast<u32x4*>(vdst + (size_t)r * HD + ch * 8) =
        valid ? *reinterpret_cast<const u32x4*>(row_at(v, vs, b, hk, key0 + r) + ch * 8) : zero;
  }
}

// The LDS word a transposing read returns: ds_read_b64_tr_b16 with lane j
// pointing at 4 consecutive FP16 values gives, in each group of 16 lanes,
// lane l the values at offset l % 4 of the 4 lanes 4e + (l % 16) / 4 of its
// group (e = 0..3): the 4 x 16 block those lanes address, read by column.
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 tr_h4;
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ h4 lds_read_tr(const char* p) {
  const tr_h4 r = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
      (__attribute__((address_space(3))) tr_h4*)(p));
  return __builtin_bit_cast(h4, r);
}

// Raw-buffer descriptor (gfx9 layout: base address, stride 0, range in
// bytes, 32-bit data format) for loads from `base`; the hardware returns
// zeros for any lane whose offset lies at or past `bytes`.
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, int bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4{(int)(uint32_t)a, (int)(uint32_t)(a >> 32), bytes, 0x00020000};
}

// One direct-to-LDS load: 64 lanes x 16 bytes from the buffer `rsrc` at byte
// offset voff (per lane) + soff (wave-uniform) into the 1 KiB of LDS at byte
// address lds_addr (wave-uniform; M0 holds it for the load). Written as
// inline assembly so that the compiler does not track these loads: it
// orders a transposing LDS read (ds_read_b64_tr_b16) after every load into
// LDS still in flight (vmcnt(0)), which would stall each MFMA step on the
// loads meant for later blocks. The attention body orders its loads and
// operand reads itself (explicit vmcnt waits before the barriers that
// publish a block). M0 is declared clobbered, so code the compiler places
// after the load never assumes M0 still holds a value it set earlier; M0 is
// a reserved register to the compiler, which warns about naming it, and the
// pragma silences that warning for this function alone.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_to_lds(i32x4 rsrc, uint32_t lds_addr, int voff, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier that also drains this wave's outstanding LDS operations,
// so LDS writes issued before it are visible to every wave after it. The
// memory clobber keeps the compiler from moving memory accesses across it,
// and the scheduling fences keep arithmetic on its own side too: the
// ping-pong schedule depends on a phase's work not leaking into the next.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Sync mode: fill n16 16-byte words at p with FP16 NaN (grid-stride).
__global__ void __launch_bounds__(256) fa_poison_kernel(u32x4* p, uint64_t n16) {
  const u32x4 nan = {NAN16X2, NAN16X2, NAN16X2, NAN16X2};
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * 256)
    p[i] = nan;
}

// Split mode's second kernel: for every query row, combines the parts'
// results O_s (normalised by the part's own row sum) and lse_s into
//   O = sum_s w_s O_s / sum_s w_s,  lse = M + ln sum_s w_s,
//   w_s = exp(lse_s - M),  M = max_s lse_s,
// the log-sum-exp algebra of the online softmax applied once across parts.
// A part whose lse is -inf (the row sees none of its keys) has weight 0 (its
// O row holds zeros); a row that sees no key at all gets O = 0 and
// lse = -inf. 32 lanes per row: lane i reads the lse of parts i, i + 32, ...,
// so the maximum and the weight sum are reductions over the 32 lanes, and
// each lane accumulates 4 of the 128 dims over all parts, with the weights
// broadcast from the lane that computed them and the O loads independent of
// each other (unrolled, so several are in flight). 8 rows per 256-thread
// block, grid-stride over the rows = B * Hq * Nq; o is written through its
// strides, lse (may be null) contiguously.
__device__ __forceinline__ float max32(float x) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 32));
  return x;
}
__device__ __forceinline__ float sum32(float x) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) x += __shfl_xor(x, m, 32);
  return x;
}
__global__ void __launch_bounds__(256) fa_merge_kernel(const float* __restrict__ opart,
                                                       const float* __restrict__ lpart,
                                                       _Float16* __restrict__ o,
                                                       float* __restrict__ lse, int splits,
                                                       int64_t rows, int heads_q, int seq_q,
                                                       Strides os) {
  const int sub = threadIdx.x & 31;
  const int64_t step = (int64_t)gridDim.x * 8;
  for (int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5); row < rows; row += step) {
    float mx = -INFINITY;
    for (int s = sub; s < splits; s += 32) mx = fmaxf(mx, lpart[s * rows + row]);
    mx = max32(mx);
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f, wsum = 0.f;
    if (mx != -INFINITY) {
      const float* col = opart + (size_t)row * HD + 4 * sub;
      const size_t pstride = (size_t)rows * HD;
      for (int s0 = 0; s0 < splits; s0 += 32) {
        const int s = s0 + sub;
        const float ls = s < splits ? lpart[s * rows + row] : -INFINITY;
        const float w = ls == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((ls - mx) * (float)LOG2E);
        wsum += w;
        const int n = min(32, splits - s0);
        auto add = [&](float wi, const float4& v) {
          a0 = __builtin_fmaf(wi, v.x, a0);
          a1 = __builtin_fmaf(wi, v.y, a1);
          a2 = __builtin_fmaf(wi, v.z, a2);
          a3 = __builtin_fmaf(wi, v.w, a3);
        };
        int i = 0;
        for (; i + 4 <= n; i += 4) {        // four loads in flight before their FMAs
          float4 v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[j] = *reinterpret_cast<const float4*>(col + (size_t)(s0 + i + j) * pstride);
#pragma unroll
          for (int j = 0; j < 4; ++j) add(__shfl(w, i + j, 32), v[j]);
        }
        for (; i < n; ++i)
          add(__shfl(w, i, 32), *reinterpret_cast<const float4*>(col + (size_t)(s0 + i) * pstride));
      }
      wsum = sum32(wsum);
    }
    const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
    const int64_t bh = row / seq_q;
    const int i = (int)(row - bh * seq_q);
    const int b = (int)(bh / heads_q), h = (int)(bh - (int64_t)b * heads_q);
    const h4 out = {(_Float16)(a0 * inv), (_Float16)(a1 * inv), (_Float16)(a2 * inv),
                    (_Float16)(a3 * inv)};
    *reinterpret_cast<h4*>(row_at(o, os, b, h, i) + 4 * sub) = out;
    if (lse && sub == 0) lse[row] = wsum > 0.f ? mx + __builtin_amdgcn_logf(wsum) * LN2 : -INFINITY;
  }
}

// The merge for few rows with many parts (decode: a dozen rows, a hundred
// parts or more), where fa_merge_kernel's cost is one row's walk over its
// parts: a 256-thread workgroup per row (grid-stride over the rows). The
// workgroup first finds the row's maximum lse; then its 8 groups of 32 lanes
// each run fa_merge_kernel's per-lane accumulation over parts g, g + 8,
// g + 16, ..., and the 8 partial sums of O and of the weights are added
// through LDS, so the walk is 8 times shorter. Same inputs, outputs and
// special cases as fa_merge_kernel; only the FP32 summation order differs.
__global__ void __launch_bounds__(256) fa_merge_wide_kernel(const float* __restrict__ opart,
                                                            const float* __restrict__ lpart,
                                                            _Float16* __restrict__ o,
                                                            float* __restrict__ lse, int splits,
                                                            int64_t rows, int heads_q, int seq_q,
                                                            Strides os) {
  constexpr int G = 8;                      // lane groups per workgroup
  __shared__ float4 part_o[G][HD / 4];
  __shared__ float part_w[G];
  __shared__ float part_m[G];
  const int sub = threadIdx.x & 31, grp = threadIdx.x >> 5;
  const size_t pstride = (size_t)rows * HD;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    float mx = -INFINITY;
    for (int s = threadIdx.x; s < splits; s += 32 * G) mx = fmaxf(mx, lpart[s * rows + row]);
    mx = max32(mx);
    if (sub == 0) part_m[grp] = mx;
    __syncthreads();
    mx = part_m[0];
#pragma unroll
    for (int g = 1; g < G; ++g) mx = fmaxf(mx, part_m[g]);
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f, wsum = 0.f;
    if (mx != -INFINITY) {
      const float* col = opart + (size_t)row * HD + 4 * sub;
      const int mine = splits > grp ? (splits - grp + G - 1) / G : 0;   // parts grp + G t
      auto add = [&](float wi, const float4& v) {
        a0 = __builtin_fmaf(wi, v.x, a0);
        a1 = __builtin_fmaf(wi, v.y, a1);
        a2 = __builtin_fmaf(wi, v.z, a2);
        a3 = __builtin_fmaf(wi, v.w, a3);
      };
      for (int t0 = 0; t0 < mine; t0 += 32) {
        const int t = t0 + sub;
        const float ls = t < mine ? lpart[(grp + G * t) * rows + row] : -INFINITY;
        const float w = ls == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((ls - mx) * (float)LOG2E);
        wsum += w;
        const int n = min(32, mine - t0);
        int i = 0;
        for (; i + 4 <= n; i += 4) {        // four loads in flight before their FMAs
          float4 v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[j] = *reinterpret_cast<const float4*>(col + (size_t)(grp + G * (t0 + i + j)) * pstride);
#pragma unroll
          for (int j = 0; j < 4; ++j) add(__shfl(w, i + j, 32), v[j]);
        }
        for (; i < n; ++i)
          add(__shfl(w, i, 32),
              *reinterpret_cast<const float4*>(col + (size_t)(grp + G * (t0 + i)) * pstride));
      }
      wsum = sum32(wsum);
    }
    part_o[grp][sub] = float4{a0, a1, a2, a3};
    if (sub == 0) part_w[grp] = wsum;
    __syncthreads();
    if (threadIdx.x < HD) {
      const int d = threadIdx.x;
      float acc = 0.f, wall = 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float4 pv = part_o[g][d >> 2];
        acc += (d & 3) == 0 ? pv.x : (d & 3) == 1 ? pv.y : (d & 3) == 2 ? pv.z : pv.w;
        wall += part_w[g];
      }
      const float inv = wall > 0.f ? 1.f / wall : 0.f;
      const int64_t bh = row / seq_q;
      const int i = (int)(row - bh * seq_q);
      const int b = (int)(bh / heads_q), h = (int)(bh - (int64_t)b * heads_q);
      row_at(o, os, b, h, i)[d] = (_Float16)(acc * inv);
      if (lse && d == 0) lse[row] = wall > 0.f ? mx + __builtin_amdgcn_logf(wall) * LN2 : -INFINITY;
    }
    __syncthreads();                        // LDS is reused by the next row
  }
}

// Trace mode: thread 0 writes the tile's record (layout at TRACE_WORDS)
// with the start stamps real0/clk0 and stamps taken now.
__device__ __forceinline__ void trace_record(const FaArgs& args, int tile, uint64_t real0,
                                             uint64_t clk0, int nblk, int bn) {
  const uint64_t real1 = __builtin_amdgcn_s_memrealtime();
  const uint64_t clk1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x != 0) return;
  // s_getreg encodings (id | offset << 6 | (size - 1) << 11): HW_ID (id 4)
  // and XCC_ID (id 20), all 32 bits.
  const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
  const uint32_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20) & 15u;
  uint64_t* rec = args.trace + (size_t)tile * TRACE_WORDS;
  rec[0] = (uint64_t)hw | ((uint64_t)xcc << 32);
  rec[1] = real0;
  rec[2] = real1;
  rec[3] = clk0;
  rec[4] = clk1;
  rec[5] = (uint64_t)tile;
  rec[6] = (uint64_t)nblk;
  rec[7] = (uint64_t)bn;
}

// Ping-pong attention body: 8 waves x 32 query rows (BM = 256), two wave
// groups of four, one wave of each group per SIMD. The key loop runs in
// phases separated by workgroup barriers; a wave alternates an MFMA step
// (S^T(j) = K(j) Q^T and O^T += V^T(j-1) P^T(j-1)) with a VALU step (online
// softmax of S(j) into P(j)), and group 1 runs one phase behind group 0, so
// on every SIMD one wave keeps the matrix pipe busy while the other does its
// softmax (the FA3 ping-pong schedule, here across the two waves of a SIMD).
//
// LDS holds a ring of NS K blocks and NS V blocks (NS >= 2). Phase pair t
// (phases 2t, 2t+1) reads K(t) and V(t-1). In phase 2t the direct-to-LDS
// loads (buffer_load_dwordx4 ... lds, 1 KiB per wave instruction) of
// K(t+NS-1) and V(t+NS-2) go out into the ring slots pair t-1 finished with:
// from group 1's VALU step (FP32 accumulator), or from group 0's MFMA step,
// one load every few MFMAs so the vector-memory issue never stalls the wave
// for long (FP16 accumulator). The issuing group waits for its pair t+2-NS
// loads before the barrier that opens pair t+1, so every load has NS-1
// phase pairs minus part of a phase to land and no VGPR or LDS write
// instruction is spent on staging.
//
// The running max is raised lazily (TAU, in log2 units): a row keeps its max
// until a block exceeds it by more than TAU, so P <= 2^TAU and the O/l
// rescale runs only on the rare blocks where some row of the wave needs it.
// With TAU = 0 the max tracks every increase (FP16 O must not grow).
// LDS ring slots of the ping-pong body, in 16-byte chunks. A K block is BN
// rows of 128 dims as they lie in memory, 17 chunks per row (16 + 1 pad). A V
// block is either V^T, the key-permuted transposed copy the prep kernel
// writes (128 dim rows of BN keys, BN / 8 + 1 chunks per row), or, in the
// tile that reads V in its natural layout (VNAT), BN key rows of 128 dims,
// 16 chunks per row with no pad: row r holds its chunk c at position
// c ^ 4 (r % 4), which spreads the 4 rows a transposing read takes its
// columns from over the 4 quarters of the banks.
constexpr int K_CHUNKS = 17;
constexpr int k_block_bytes(int bn) { return bn * K_CHUNKS * 16; }
constexpr int v_block_bytes(int bn, bool vnat) { return vnat ? bn * HD * 2 : HD * (bn / 8 + 1) * 16; }

template <bool ACC16, int BN, int NS, int MODE, bool PACKED, bool VNAT>
__device__ __forceinline__ void fa_pp_tile(const FaArgs& args, const int tile, const int split) {
  constexpr bool CAPTURE = MODE == MODE_CAPTURE;
  constexpr bool TRACE = MODE == MODE_TRACE;
  constexpr bool SYNC = MODE == MODE_SYNC;
  constexpr bool SPLIT = MODE == MODE_SPLIT;
  uint64_t real0 = 0, clk0 = 0;
  if constexpr (TRACE) {
    real0 = __builtin_amdgcn_s_memrealtime();
    clk0 = __builtin_amdgcn_s_memtime();
  }
  const _Float16* __restrict__ q = args.q;
  const _Float16* __restrict__ k = args.k;
  const _Float16* __restrict__ v = args.v;
  _Float16* __restrict__ o = args.o;
  const int heads_q = args.heads_q, group = args.group, seq_q = args.seq_q, seq_k = args.seq_k;
  const int nk_valid = args.nk_valid;
  const float c = args.c;
  constexpr int NT = 512;
  constexpr int BM = 256;
  constexpr int KT = BN / 32;            // 32-key S^T tiles per block
  constexpr int KS = BN / 16;            // 16-key PV steps per block
  constexpr int NQK = 8 * KT;            // QK MFMAs per block
  constexpr int NPV = 4 * KS;            // PV MFMAs per block
  static_assert(NQK == NPV, "QK and PV MFMA counts pair up");
  // Padded K and V^T rows keep every operand address "lane base + immediate"
  // and spread a read over the banks: the extra chunk per row makes the 32
  // rows a wave reads at one chunk column (ds_read_b128) hit distinct bank
  // groups. Natural V rows are swizzled instead (v_block_bytes): each
  // half-wave of a transposing read addresses 4 rows x 64 bytes, which the
  // swizzle puts in the 4 distinct quarters of the 64 banks.
  constexpr int KROW = K_CHUNKS * 16;                  // bytes per K row
  constexpr int VCH = VNAT ? HD / 8 : BN / 8 + 1;      // chunks per V (or V^T) row
  constexpr int VDATA = VNAT ? HD / 8 : BN / 8;        // of which data chunks
  constexpr int VROW = VCH * 16;                       // bytes per V (or V^T) row
  constexpr int KBYTES = k_block_bytes(BN);
  constexpr int VBYTES = v_block_bytes(BN, VNAT);
  // Direct-to-LDS loads fill 1 KiB of consecutive LDS per wave instruction,
  // pad chunks included (they receive a harmless copy of chunk 0 of the row).
  constexpr int KI = KBYTES / 1024;      // DMA instructions per K block
  constexpr int VI = VBYTES / 1024;      // DMA instructions per V block
  constexpr int NI = KI + VI;            // per phase pair, spread over group 0
  constexpr int NIW = (NI + 3) / 4;      // most instructions one group-0 wave issues
  static_assert(KBYTES == KI * 1024 && VBYTES == VI * 1024, "blocks are whole DMA instructions");
  constexpr int PF = 4;                  // LDS operand prefetch depth (MFMAs)
  constexpr float TAU = ACC16 ? 0.f : 8.f;

  extern __shared__ __attribute__((aligned(16))) char lds[];
  char* kbase = lds;                     // NS K blocks
  char* vbase = lds + NS * KBYTES;       // NS V blocks

  // The thread index passes through an opaque move, so nothing derived from
  // it is hoisted out of the work-queue loop around this function: values a
  // tile can recompute in a few instructions would otherwise stay live in
  // registers across every tile's key loop.
  int tid;
  asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hf = lane >> 5;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);   // provably wave-uniform
  // Role: which phase parity this wave's MFMA steps fall on. Waves w and w+4
  // share a SIMD (round-robin wave placement, read back from HW_ID).
  const int grp = wave_u >> 2;

  // A tile is 256 consecutive rows of a row sequence. Unpacked, a sequence
  // is the Nq query rows of one (batch, query head). Packed (PACKED,
  // grouped-query attention with few query rows), it is the Nq * group rows
  // of one (batch, KV head) in position-major order: row r is position
  // r / group of query head kv_head * group + r % group, so the heads that
  // share K and V fill one tile instead of a tile each. Every row computes
  // exactly what it computes unpacked (the key loop and its rounding are
  // per row). A tile may run past the sequence (a ragged last tile): its
  // rows past the end compute on a copy of the last row and store nothing.
  // Without a mask, consecutive tile indices walk the tiles of one sequence;
  // with the causal mask, whose tiles differ in work, they walk the
  // sequences at one tile position, the tiles with the most key blocks
  // first, so the short tiles are taken last.
  constexpr bool packed = PACKED;
  const int seq_r = packed ? seq_q * group : seq_q;     // rows per sequence
  const int tiles_q = (seq_r + BM - 1) / BM;
  const int nbh = args.tiles / tiles_q;                  // sequences
  int bh, qt;
  if (args.causal) {
    const int r = tile / nbh;
    bh = tile - r * nbh;
    qt = tiles_q - 1 - r;
  } else {
    bh = tile / tiles_q;
    qt = tile - bh * tiles_q;
  }
  const int heads_kv = heads_q / group;
  const int b = bh / (packed ? heads_kv : heads_q);
  const int hs = bh - b * (packed ? heads_kv : heads_q);  // the sequence's head (KV head if packed)
  const int hk = packed ? hs : hs / group;                // KV head
  const size_t kv = (size_t)b * heads_kv + hk;
  const _Float16* kp = row_at(k, args.ks, b, hk, 0);
  // This KV head's V rows (natural layout) or V^T rows (128 rows of seq_k keys).
  const _Float16* vp = VNAT ? row_at(v, args.vs, b, hk, 0) : v + kv * (size_t)HD * seq_k;
  // Query head and position of row r of the sequence.
  auto head_of = [&](int r) { return packed ? hk * group + r % group : hs; };
  auto pos_of = [&](int r) { return packed ? r / group : r; };
  const int row = qt * BM + wave_u * 32 + l32;          // this lane's row of the sequence
  const bool row_ok = row < seq_r;
  const int rowc = row_ok ? row : seq_r - 1;            // the row it loads
  const size_t rows_all = (size_t)(packed ? nbh * group : nbh) * seq_q;   // B * Hq * Nq
  // Its index in [B * Hq * Nq] (lse, statistics, split parts).
  const size_t grow = ((size_t)b * heads_q + head_of(rowc)) * seq_q + pos_of(rowc);
  const int krow = (int)(args.ks.n * 2);                 // K row pitch in bytes
  const int vrow = VNAT ? (int)(args.vs.n * 2) : seq_k * 2;   // V (or V^T) row pitch in bytes

  // Last key this lane's row sees (klim) and the smallest such limit over the
  // wave (klim_w, wave-uniform: the wave's first row); blocks reaching past
  // klim_w take the key loop's masked part. With the causal mask the workgroup streams only the
  // key blocks its last row sees.
  int nblk = seq_k / BN;
  int klim = nk_valid - 1, klim_w = nk_valid - 1;
  if (args.causal) {
    klim = min(klim, pos_of(row) + args.causal_off);
    klim_w = min(klim_w, pos_of(qt * BM + wave_u * 32) + args.causal_off);
    // Keys [0, kend) are seen by the tile's last row.
    const int kend = pos_of(min(qt * BM + BM, seq_r) - 1) + 1 + args.causal_off;
    nblk = kend <= 0 ? 0 : min(nblk, (kend + BN - 1) / BN);
  }
  // Split mode: this work item streams key blocks [kb0, kb1) of the tile
  // (part `split` of args.splits near-equal parts of the key blocks), with
  // the loads, limits and masks below relative to key kb0 * BN.
  int kb0 = 0;
  if constexpr (SPLIT) {
    const int nbt = seq_k / BN;
    kb0 = (int)((int64_t)split * nbt / args.splits);
    const int kb1 = (int)((int64_t)(split + 1) * nbt / args.splits);
    nblk = max(0, min(nblk, kb1) - kb0);
    klim -= kb0 * BN;
    klim_w -= kb0 * BN;
  }
  const size_t part = (size_t)split * rows_all + grow;   // split mode: partial row
  if (nblk == 0) {
    // No row of this tile sees a key (bottom-right mask, Nq > Nk): O = 0 and
    // lse = -inf. Uniform over the workgroup, before any barrier or load.
    if constexpr (CAPTURE) {
      if (hf == 0 && row_ok) {
        const size_t rows = rows_all, nb = seq_k / BN;
        for (size_t j = 0; j < nb; ++j) {
          args.stats[(0 * nb + j) * rows + grow] = -INFINITY;
          args.stats[(1 * nb + j) * rows + grow] = 0.f;
          args.stats[(2 * nb + j) * rows + grow] = 1.f;
          args.stats[(3 * nb + j) * rows + grow] = 0.f;
        }
      }
    }
    if constexpr (TRACE) trace_record(args, tile, real0, clk0, 0, BN);
    if (!row_ok) return;
    if constexpr (SPLIT) {
      // The part's lse is -inf and its O row zeros (weight 0 in the merge).
      if (hf == 0) args.lpart[part] = -INFINITY;
      float* prow = args.opart + part * HD;
      const float4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) *reinterpret_cast<float4*>(prow + dt * 32 + 8 * g + 4 * hf) = zero;
      return;
    }
    if (args.lse && hf == 0) args.lse[grow] = -INFINITY;
    const h4 zero = {(_Float16)0.f, (_Float16)0.f, (_Float16)0.f, (_Float16)0.f};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<h4*>(row_at(o, args.os, b, head_of(rowc), pos_of(rowc)) + dt * 32 +
                               8 * g + 4 * hf) = zero;
    return;
  }

  h8 qf[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    qf[kk] = *reinterpret_cast<const h8*>(row_at(q, args.qs, b, head_of(rowc), pos_of(rowc)) +
                                          kk * 16 + hf * 8);

  // Group-0 wave dw issues DMA instructions q = dw + 4m (m < NIW, q < NI);
  // q < KI is K instruction q, otherwise V instruction q - KI. The per-lane
  // source offset inside a block is fixed, so it is computed once. Natural V
  // instruction q' fills rows 4q' .. 4q' + 3 with no pad chunks, so all of
  // them share one per-lane offset (vdma: row lane / 16 of the four, the
  // chunk its swizzled position holds) and differ by 4q' rows, a scalar.
  const int dw = wave_u & 3;
  constexpr int NKW = (KI + 3) / 4;      // most K instructions one wave issues
  constexpr int NOFF = VNAT ? NKW : NIW;  // per-lane offsets kept
  const int vdma = (lane >> 4) * vrow + ((lane & 15) ^ (4 * ((lane >> 4) & 3))) * 16;
  int dma_off[NOFF];
#pragma unroll
  for (int m = 0; m < NOFF; ++m) {
    const int q = dw + 4 * m;
    if (q < KI) {
      const int i = q * 64 + lane, r = i / 17, ch = i % 17;
      dma_off[m] = r * krow + (ch < 16 ? ch : 0) * 16;
    } else if constexpr (VNAT) {
      dma_off[m] = vdma;
    } else {
      const int i = (q - KI) * 64 + lane, r = i / VCH, ch = i % VCH;
      dma_off[m] = r * vrow + (ch < VDATA ? ch : 0) * 16;
    }
  }
  // The loads are buffer loads through one descriptor per operand (base =
  // this KV head's K or V, range = the bytes its seq_k rows span, so the
  // hardware bounds-checks every lane): the per-lane offset is dma_off, the
  // block offset a wave-uniform scalar (see dma_to_lds).
  const i32x4 krsrc = buffer_rsrc(kp + (size_t)kb0 * BN * args.ks.n, (seq_k - kb0 * BN - 1) * krow + HD * 2);
  const i32x4 vrsrc = VNAT ? buffer_rsrc(vp + (size_t)kb0 * BN * args.vs.n, (seq_k - kb0 * BN - 1) * vrow + HD * 2)
                           : buffer_rsrc(vp + kb0 * BN, seq_k * (HD * 2) - kb0 * (BN * 2));
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  // DMA instruction m of this wave for K block kb -> ring slot ks and V
  // block vb -> slot vs. Branch free: the K/V choice is a select on
  // wave-uniform values; only a wave's last instruction can be absent.
  auto dma_one = [&](int m, int kb, int ks, int vb, int vs) {
    const int q = dw + 4 * m;
    if (m == NIW - 1 && NI % 4 != 0 && q >= NI) return;
    const bool isk = q < KI;
    const int dst = isk ? ks * KBYTES + q * 1024 : NS * KBYTES + vs * VBYTES + (q - KI) * 1024;
    const int soff = isk ? kb * (BN * krow) : VNAT ? (vb * BN + 4 * (q - KI)) * vrow : vb * (BN * 2);
    dma_to_lds(isk ? krsrc : vrsrc, lds0 + dst, m < NOFF ? dma_off[m] : vdma, soff);
  };
  auto issue = [&](int kb, int ks, int vb, int vs) {
#pragma unroll
    for (int m = 0; m < NIW; ++m) dma_one(m, kb, ks, vb, vs);
  };
  // Wait until at most n of this wave's DMA loads are outstanding.
  auto wait_dma = [&](int n) {
    __builtin_amdgcn_sched_barrier(0);
    switch (n) {
      case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
      case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
      case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
      case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
      case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
      case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
      case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
      case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
      case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
      case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
      case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
      case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
      case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
      case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
      case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
      case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
      case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
      case 17: asm volatile("s_waitcnt vmcnt(17)" ::: "memory"); break;
      case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
      case 19: asm volatile("s_waitcnt vmcnt(19)" ::: "memory"); break;
      case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
      case 21: asm volatile("s_waitcnt vmcnt(21)" ::: "memory"); break;
      case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
      case 23: asm volatile("s_waitcnt vmcnt(23)" ::: "memory"); break;
      default: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert((NS - 2) * NIW <= 24 && NS >= 2, "wait_dma covers at most 24 loads");
  // MFMA index after which DMA instruction m is issued inside an MFMA step.
  constexpr int DSTEP = (2 * NQK - 8) / NIW > 0 ? (2 * NQK - 8) / NIW : 1;
  static_assert(1 + DSTEP * (NIW - 1) < 2 * NQK, "every DMA instruction finds an MFMA slot");
  static_assert(NIW <= 8 * KT, "every DMA instruction finds an exponential pair of a VALU step");

  f32x16 acc[4];
  f32x16 s[KT];
  h8 p[KS];
  float m = NEG_BIG, lsum = 0.f;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x16{};
  // FP16 accumulator: O is an FP16 value at every packet boundary. The
  // matrix cores accumulate a packet's PV products (rescaled like the FP32
  // accumulator when the max moves) on top of it in the FP32 registers, and
  // at the packet's end the sum is rounded to FP16 in place -- the merge
  // O16 = fp16(alpha O16 + partial) of the reference's FP16-O kernel, once
  // per 512 keys, its packet (there: the partial rounded to FP16 first, and
  // an FP16 alpha). An O beyond the FP16 range becomes inf, as there.
  constexpr int PACKET = 512 / BN;       // key blocks per packet
  auto round_acc_fp16 = [&]() {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const h2 t = {(_Float16)acc[dt][i], (_Float16)acc[dt][i + 1]};
        acc[dt][i] = (float)t[0];
        acc[dt][i + 1] = (float)t[1];
      }
  };
#pragma unroll
  for (int i = 0; i < KS; ++i) p[i] = h8{};

  // Per-lane operand offsets. QK op (t, kk) reads K row 32t + l32, chunk
  // 2kk + hf. PV op (dt, ks) needs, for dim 32dt + l32, the keys 16ks + 4hf
  // + {0..3} and + {8..11}: from V^T, row 32dt + l32, chunk 2ks + hf (one
  // 16-byte read); from natural V, two transposing reads, in which lane j =
  // 16g + 4e + i (g = j / 16) points at V row 16ks + 4(g / 2) + e (+ 8 for the
  // second), dims 32dt + 16(g % 2) + 4i .. + 3: chunk 4dt + 2(g % 2) + i / 2,
  // stored at position 4(dt ^ e) + 2(g % 2) + i / 2 of a row with r % 4 = e.
  // That position depends on dt and on the lane, so natural V keeps one
  // base per dt.
  const int k_lane = l32 * KROW + hf * 16;
  const int v_lane = l32 * VROW + hf * 16;
  int v_nat[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const int e = (lane & 15) >> 2;
    v_nat[dt] = (4 * hf + e) * VROW + (4 * (dt ^ e) + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)) * 16 +
                (lane & 1) * 8;
  }

  // MFMA step for block j: S^T(j) = K(j) Q^T and O^T += V^T(j-1) P^T(j-1),
  // QK and PV MFMAs interleaved, operands prefetched PF MFMAs ahead.
  // Operand i of a step: QK op n = i / 2 (even i) covers S tile n % KT at
  // k-step n / KT, so consecutive QK ops alternate accumulators; with PV ops
  // in between, no accumulator is reused within four MFMAs and dependent
  // MFMAs never wait on each other.
  auto ld = [&](const char* kb, const char* vb, int i) -> h8 {
    const int n = i >> 1;
    if ((i & 1) == 0) {
      const int t = n % KT, kk = n / KT;
      return *reinterpret_cast<const h8*>(kb + k_lane + t * 32 * KROW + kk * 32);
    }
    const int dt = n % 4, ks = n / 4;
    if constexpr (VNAT) {
      const char* at = vb + v_nat[dt] + ks * 16 * VROW;
      return __builtin_shufflevector(lds_read_tr(at), lds_read_tr(at + 8 * VROW), 0, 1, 2, 3, 4, 5, 6,
                                     7);
    } else {
      return *reinterpret_cast<const h8*>(vb + v_lane + dt * 32 * VROW + ks * 32);
    }
  };
  // The step's first PF operands. A group-1 wave reads them at the end of
  // the VALU step before its MFMA step (its blocks were published one phase
  // earlier), so its MFMA step starts without waiting for LDS; a group-0
  // step reads them itself.
  h8 fr[PF];
  auto preload = [&](const char* kb, const char* vb) {
#pragma unroll
    for (int i = 0; i < PF; ++i) fr[i] = ld(kb, vb, i);
  };
  auto mfma_step = [&](const char* kb, const char* vb, bool with_dma, int dkb, int dks, int dvb,
                       int dvs, auto preloaded) {
    if constexpr (!decltype(preloaded)::value) preload(kb, vb);
#pragma unroll
    for (int i = 0; i < 2 * NQK; ++i) {
      const h8 a = fr[i % PF];
      const int n = i >> 1;
      // The first product into each S tile starts from a zero accumulator
      // operand instead of zeroed registers.
      if ((i & 1) == 0) {
        s[n % KT] = mfma32(a, qf[n / KT], n < KT ? f32x16{} : s[n % KT]);
      } else {
        acc[n % 4] = mfma32(a, p[n / 4], acc[n % 4]);
      }
      if (i + PF < 2 * NQK) fr[i % PF] = ld(kb, vb, i + PF);
      if (i >= 1 && (i - 1) % DSTEP == 0 && (i - 1) / DSTEP < NIW) {
        if (with_dma) dma_one((i - 1) / DSTEP, dkb, dks, dvb, dvs);
      }
      // Keep source order: operand reads stay PF MFMAs ahead of their use.
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  if constexpr (SYNC) {
    // Poison the whole ring (every K and V slot, row pads included), so an
    // operand read of LDS that no load of this tile has written is a NaN.
    for (int i = tid; i < NS * (KBYTES + VBYTES) / 16; i += NT)
      reinterpret_cast<u32x4*>(lds)[i] = u32x4{NAN16X2, NAN16X2, NAN16X2, NAN16X2};
    lds_barrier();
  }
  // V slot NS-1 (read as "V(-1)" by the first MFMA step) starts as zeros:
  // the first step multiplies it by P = 0.
  for (int i = tid; i < VBYTES / 16; i += NT)
    reinterpret_cast<u32x4*>(vbase + (NS - 1) * VBYTES)[i] = u32x4{0u, 0u, 0u, 0u};

  const int last = nblk - 1;
  // Prologue (group 0): K(0..NS-2) -> slots 0..NS-2 and V(0..NS-3) -> slots
  // 0..NS-3, everything pairs before pair 0 would have loaded. Block indices
  // past the end are clamped, so every pair issues the same loads and the
  // fixed wait counts stay exact. (issue() always loads one K and one V
  // block; the prologue's extra V loads target slots that are rewritten
  // before use.)
  if (grp == 0) {
#pragma unroll
    for (int i = 0; i + 1 < NS; ++i) issue(min(i, last), i, min(i, last), i);
  }
  wait_dma(0);
  // Every load of this wave has landed, the Q fragments included. Consuming
  // them here tells the compiler so: it does not see the wait above (inline
  // assembly), and would otherwise wait for the Q loads, and with them for
  // every later load of the wave, before the first QK products of each key
  // block.
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) asm volatile("" ::"v"(qf[kk]));
  lds_barrier();

  // VALU step: online softmax of S(j) into P(j). For the FP16 accumulator,
  // when block j starts a packet, acc holds the previous packet's PV products
  // (the last of them added by MFMA step j): it is rounded to FP16 first.
  // at(i) runs before the exponentials of score pair i (0 <= i < 8 KT), the
  // points at which a step that issues loads spreads them.
  auto valu_step = [&](int key0, auto masked, auto&& at) {
    if constexpr (ACC16) {
      const int j = key0 / BN;
      if (j > 0 && j % PACKET == 0) round_acc_fp16();
    }
    // Keys past the row's limit (zero padding of a ragged last block, keys
    // beyond the causal diagonal) get MASKED added to their score, so P = 0.
    // S^T register r of lane half hf holds key 32t + 8(r / 4) + 4hf + r % 4
    // of the block. The penalty weight clamp(key - limit, 0, 1) is computed
    // in float arithmetic: a per-element compare and select would hold up to
    // 64 lane masks in scalar registers, and that pressure spills scalar
    // registers across the whole key loop.
    if constexpr (decltype(masked)::value) {
      const int lim = klim - key0 - 4 * hf;
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float d = (float)(32 * t + 8 * (r >> 2) + (r & 3) - lim);
          s[t][r] = __builtin_fmaf(__builtin_amdgcn_fmed3f(d, 0.f, 1.f), MASKED, s[t][r]);
        }
    }
    // Row max as a balanced 3-ary tree of v_maximum3 (independent maxima
    // issue back to back; a running max would be one long dependent chain).
    float mv[KT * 16];
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mv[16 * t + r] = s[t][r];
#pragma unroll
    for (int n = KT * 16; n > 1; n = (n + 2) / 3) {
#pragma unroll
      for (int i = 0; 3 * i < n; ++i) {
        float x = mv[3 * i];
        if (3 * i + 1 < n) x = smax(x, mv[3 * i + 1]);
        if (3 * i + 2 < n) x = smax(x, mv[3 * i + 2]);
        mv[i] = x;
      }
    }
    const float mx = half_max(mv[0]);
    const bool need = (mx - m) * c > TAU;
    float alpha = 1.f;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float mnew = need ? smax(m, mx) : m;
      alpha = __builtin_amdgcn_exp2f((m - mnew) * c);
      m = mnew;
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc[dt] *= alpha;
    }
    const float mc = m * c;
    // Row sum in four independent partial sums of the FP16-rounded P the PV
    // products use, so numerator and denominator use identical weights: one
    // mixed-precision add per value (add_f16), on the plain VALU pipe.
    float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < KT; ++t) {
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        h8 frag;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          at((2 * t + g2) * 4 + e / 2);
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][8 * g2 + e], c, -mc));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][8 * g2 + e + 1], c, -mc));
          const h2 pr = {(_Float16)p0, (_Float16)p1};
          frag[e] = pr[0];
          frag[e + 1] = pr[1];
          ls[e >> 1] = add_f16<0>(ls[e >> 1], pr);
          ls[(e >> 1) ^ 2] = add_f16<1>(ls[(e >> 1) ^ 2], pr);
        }
        p[2 * t + g2] = frag;
      }
    }
    const float zsum = (ls[0] + ls[1]) + (ls[2] + ls[3]);
    lsum += zsum;
    if constexpr (CAPTURE) {         // capture mode: this block's row statistics
      const float z = half_sum(zsum), lrow = half_sum(lsum);
      if (hf == 0 && row_ok) {
        const size_t rows = rows_all;   // B * Hq * Nq
        const size_t nb = seq_k / BN, j = key0 / BN;
        float* st = args.stats + grow;
        st[(0 * nb + j) * rows] = m == NEG_BIG ? -INFINITY : m * c * LN2;
        st[(1 * nb + j) * rows] = lrow;
        st[(2 * nb + j) * rows] = alpha;
        st[(3 * nb + j) * rows] = z;
      }
    }
  };
  auto next = [](int sl) { return sl == NS - 1 ? 0 : sl + 1; };
  auto prev = [](int sl) { return sl == 0 ? NS - 1 : sl - 1; };
  auto kslot = [&](int sl) { return kbase + sl * KBYTES; };
  auto vslot = [&](int sl) { return vbase + sl * VBYTES; };
  // Loads of later pairs a group-0 wave may leave in flight at its wait:
  // (NS - 2) pairs' worth, counted for the waves that issue one instruction
  // fewer when NI is not a multiple of 4. The others then also wait for
  // their oldest load of pair j+1, issued a phase pair earlier. A constant
  // count makes the wait one s_waitcnt (a per-wave count cost a branch
  // chain in every iteration).
  constexpr int keep = (NS - 2) * (NI % 4 != 0 ? NIW - 1 : NIW);

  // Phase 2j + grp is this wave's MFMA step for block j, phase 2j + grp + 1
  // its VALU step; both groups pass the same 2 * nblk + 2 barriers. sl is
  // j % NS, the ring slot of K(j); V(j-1) sits in slot (j - 1) % NS. Pair j
  // loads K(j+NS-1) into slot (j-1) % NS and V(j+NS-2) into slot (j-2) % NS,
  // the slots pair j-1 finished with.
  // Each wave runs its key loop in two parts: blocks j < nfull, which every
  // row of the wave sees whole, with no mask code at all, then the rest
  // (the ragged tail, the causal diagonal), which always applies the
  // per-element mask. A wave-uniform test inside one loop measured 1-3%
  // slower than no test, even when never taken.
  const std::integral_constant<bool, false> unmasked, loads;
  const std::integral_constant<bool, true> masked, preloaded;
  const int nfull = klim_w + 1 < BN ? 0 : min(nblk, (klim_w + 1) / BN);
  int sl = 0;
  // Who issues the loads. Pair t's loads, K(t+NS-1) -> slot (t-1) % NS and
  // V(t+NS-2) -> slot (t-2) % NS, go out in phase 2t (pair 0's in phase 0),
  // either from group 0's MFMA step or from group 1's VALU step, which runs
  // in the same phase and has time to spare while the FP32 softmax runs: the
  // MFMA steps then carry no load issue (+0.5% at c2/c3). The FP16
  // accumulator's VALU step also rounds O every fourth block and has no time
  // to spare (there the move measured 1.7% slower), so its loads stay with
  // group 0. The wave that issues a pair's loads also waits for them, at the
  // end of the phase before the loaded blocks are read.
  constexpr bool LOADS_IN_VALU = !ACC16;
  // A wave whose 32 rows all lie past the row sequence (in a ragged last
  // tile, or a packed decode tile of a few rows) computes nothing anyone
  // reads: it skips its MFMA and VALU steps but issues its share of every
  // pair's loads, in the phase its group issues them, waits for them where
  // its group does and passes the same 2 * nblk + 2 barriers, so the ring
  // schedule is that of the full tile. The other wave of its SIMD then runs
  // its steps alone. Wave 0 always holds a row.
  const bool idle = qt * BM + wave_u * 32 >= seq_r;
  if (idle) {
    if (grp == 0) {
      for (int j = 0; j < nblk; ++j) {
        const int sp = prev(sl);
        if constexpr (!LOADS_IN_VALU) {           // phase 2j: pair j's loads
          issue(min(j + NS - 1, last), sp, min(j + NS - 2, last), prev(sp));
          if constexpr (SYNC) wait_dma(0);
        }
        lds_barrier();
        if constexpr (!LOADS_IN_VALU) wait_dma(keep);   // phase 2j + 1
        lds_barrier();
        sl = next(sl);
      }
      lds_barrier();                           // phase 2 nblk
      lds_barrier();                           // phase 2 nblk + 1
    } else {
      if constexpr (LOADS_IN_VALU) {           // phase 0: pair 0's loads
        issue(min(NS - 1, last), NS - 1, min(NS - 2, last), NS - 2);
        if constexpr (SYNC) wait_dma(0);
      }
      lds_barrier();
      for (int j = 0; j < nblk; ++j) {
        if constexpr (LOADS_IN_VALU) wait_dma(keep);   // phase 2j + 1
        lds_barrier();
        if constexpr (LOADS_IN_VALU) {         // phase 2j + 2: pair j + 1's loads
          issue(min(j + NS, last), sl, min(j + NS - 1, last), prev(sl));
          if constexpr (SYNC) wait_dma(0);
        }
        lds_barrier();
        sl = next(sl);
      }
      lds_barrier();                           // phase 2 nblk + 1
    }
  } else if (grp == 0) {
    auto pair = [&](int j, auto mask) {
      const int sp = prev(sl);
      mfma_step(kslot(sl), vslot(sp), !LOADS_IN_VALU, min(j + NS - 1, last), sp,
                min(j + NS - 2, last), prev(sp), loads);   // phase 2j: pair j starts
      if constexpr (SYNC && !LOADS_IN_VALU) wait_dma(0);   // sync mode: loads land in their phase
      lds_barrier();
      valu_step(j * BN, mask, [](int) {});   // phase 2j + 1
      if constexpr (!LOADS_IN_VALU) wait_dma(keep);        // K(j+1), V(j) have landed
      lds_barrier();
      sl = next(sl);
    };
    int j = 0;
    for (; j < nfull; ++j) pair(j, unmasked);
    for (; j < nblk; ++j) pair(j, masked);
    mfma_step(kslot(sl), vslot(prev(sl)), false, 0, 0, 0, 0, loads);   // phase 2 nblk: PV(nblk - 1)
    lds_barrier();
    lds_barrier();                           // phase 2 nblk + 1: idle
  } else {
    if constexpr (LOADS_IN_VALU) {       // phase 0: pair 0's loads
      issue(min(NS - 1, last), NS - 1, min(NS - 2, last), NS - 2);
      if constexpr (SYNC) wait_dma(0);
    }
    preload(kslot(0), vslot(NS - 1));  // phase 0: this group idles
    lds_barrier();
    auto pair = [&](int j, auto mask) {
      mfma_step(kslot(sl), vslot(prev(sl)), false, 0, 0, 0, 0, preloaded);   // phase 2j + 1
      if constexpr (LOADS_IN_VALU) wait_dma(keep);         // K(j+1), V(j) have landed
      lds_barrier();
      // Pair j + 1's loads, K(j+NS) -> slot sl and V(j+NS-1) -> prev(sl),
      // spread over the step's exponentials (in a burst at its start they
      // measured slower and fetched 4x the bytes from beyond L2).
      const int kb = min(j + NS, last), ks = sl, vb = min(j + NS - 1, last), vs = prev(sl);
      valu_step(j * BN, mask, [&](int i) {
        if constexpr (LOADS_IN_VALU) {
#pragma unroll
          for (int mi = 0; mi < NIW; ++mi)
            if (mi * (8 * KT) / NIW == i) {
              __builtin_amdgcn_sched_barrier(0);
              dma_one(mi, kb, ks, vb, vs);
              __builtin_amdgcn_sched_barrier(0);
            }
        }
      });                            // phase 2j + 2
      if constexpr (LOADS_IN_VALU && SYNC) wait_dma(0);
      // K(j+1) and V(j), the next step's blocks, were published at this
      // phase's barrier, and no load writes their slots before pair j + 2.
      preload(kslot(next(sl)), vslot(sl));
      lds_barrier();
      sl = next(sl);
    };
    int j = 0;
    for (; j < nfull; ++j) pair(j, unmasked);
    for (; j < nblk; ++j) pair(j, masked);
    mfma_step(kslot(sl), vslot(prev(sl)), false, 0, 0, 0, 0, preloaded);   // phase 2 nblk + 1: PV(nblk - 1)
    lds_barrier();
  }
  // No DMA may still be writing this workgroup's LDS when it exits.
  wait_dma(0);
  if constexpr (TRACE) trace_record(args, tile, real0, clk0, nblk, BN);

  if constexpr (CAPTURE) {
    // Key blocks past the causal diagonal leave every statistic unchanged.
    const float lrow = half_sum(lsum);
    if (hf == 0 && row_ok) {
      const size_t rows = rows_all, nb = seq_k / BN;
      for (size_t j = nblk; j < nb; ++j) {
        args.stats[(0 * nb + j) * rows + grow] = m == NEG_BIG ? -INFINITY : m * c * LN2;
        args.stats[(1 * nb + j) * rows + grow] = lrow;
        args.stats[(2 * nb + j) * rows + grow] = 1.f;
        args.stats[(3 * nb + j) * rows + grow] = 0.f;
      }
    }
  }

  // FP16 accumulator: the last (possibly partial) packet's merge.
  if constexpr (ACC16) round_acc_fp16();

  // Epilogue: O / l -> FP16 and the row's log-sum-exp
  // ln(l) + scale * m = (log2(l) + c * m) * ln 2, for rows inside Nq. A row
  // that saw no key (causal mask) has l = 0: O = 0 and lse = -inf.
  const float l = half_sum(lsum);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (!row_ok) return;
  if constexpr (SPLIT) {
    // This part's O / l in FP32 and its log-sum-exp (-inf, with O = 0, for a
    // row that sees no key of the part).
    if (hf == 0) args.lpart[part] = (__builtin_amdgcn_logf(l) + m * c) * LN2;
    float* prow = args.opart + part * HD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 val = {acc[dt][4 * g] * inv, acc[dt][4 * g + 1] * inv, acc[dt][4 * g + 2] * inv,
                            acc[dt][4 * g + 3] * inv};
        *reinterpret_cast<float4*>(prow + dt * 32 + 8 * g + 4 * hf) = val;
      }
    return;
  }
  if (args.lse && hf == 0) args.lse[grow] = (__builtin_amdgcn_logf(l) + m * c) * LN2;
  _Float16* orow = row_at(o, args.os, b, head_of(rowc), pos_of(rowc));
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      h4 out;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        out[e] = (_Float16)(acc[dt][4 * g + e] * inv);
      }
      *reinterpret_cast<h4*>(orow + dt * 32 + 8 * g + 4 * hf) = out;
    }
  }
}

// The attention kernel is persistent: a launch has one workgroup per CU (the
// LDS ring allows no second one), and each workgroup takes query tiles from a
// shared counter until none are left. The 8 accelerator dies run at clocks
// that differ by up to ~10% under the board's power limit; with a fixed
// tile-to-workgroup mapping every die gets the same number of tiles and the
// launch ends with the slowest one, while from a shared counter the faster
// dies take more tiles. Every workgroup leaves once the counter passes the
// tile count, so the grid drains. The counter lives in the workspace and is
// zeroed by the prep kernel, which runs first on the same stream. A launch
// with no more work items than CUs has one workgroup per item (the grid is
// never larger than the item count), and then each workgroup takes item
// blockIdx.x without the counter, so such a launch needs no counter reset.
// Copy of the kernel arguments read from the kernel-argument segment at
// address `addr` (scalar loads), field by field.
typedef const FaArgs __attribute__((address_space(4)))* KernargArgs;
__device__ __forceinline__ Strides load_strides(const Strides __attribute__((address_space(4)))& s) {
  return Strides{s.b, s.h, s.n};
}
__device__ __forceinline__ FaArgs load_args(uint64_t addr) {
  KernargArgs a = reinterpret_cast<KernargArgs>(addr);
  FaArgs r;
  r.q = a->q;
  r.k = a->k;
  r.v = a->v;
  r.o = a->o;
  r.lse = a->lse;
  r.stats = a->stats;
  r.trace = a->trace;
  r.next_tile = a->next_tile;
  r.tiles = a->tiles;
  r.heads_q = a->heads_q;
  r.group = a->group;
  r.seq_q = a->seq_q;
  r.seq_k = a->seq_k;
  r.nk_valid = a->nk_valid;
  r.causal = a->causal;
  r.causal_off = a->causal_off;
  r.c = a->c;
  r.qs = load_strides(a->qs);
  r.ks = load_strides(a->ks);
  r.os = load_strides(a->os);
  r.opart = a->opart;
  r.lpart = a->lpart;
  r.splits = a->splits;
  r.vs = load_strides(a->vs);
  return r;
}

template <bool ACC16, int BN, int NS, int MODE, bool PACKED, bool VNAT>
__device__ __forceinline__ void fa_pp_body(const FaArgs& args) {
  __shared__ int claimed;
  // Work items: query tiles, or in split mode (tile, part) pairs, the parts
  // of one tile consecutive.
  int items = args.tiles;
  if constexpr (MODE == MODE_SPLIT) items *= args.splits;
  const bool direct = items <= (int)gridDim.x;   // one workgroup per item
  for (int n = 0;; ++n) {
    if (direct) {
      if (n > 0) break;
    } else if (threadIdx.x == 0) {
      claimed = atomicAdd(args.next_tile, 1);
    }
    __syncthreads();
    const int item = direct ? (int)blockIdx.x : __builtin_amdgcn_readfirstlane(claimed);
    if (item >= items) break;
    int tile = item, split = 0;
    if constexpr (MODE == MODE_SPLIT) {
      tile = item / args.splits;
      split = item - tile * args.splits;
    }
    // Each tile reloads the arguments from the kernel-argument segment
    // through an address the compiler cannot follow across iterations: kept
    // from one tile to the next, all of them would stay live in scalar
    // registers across every key loop, and at 256 VGPRs per wave that
    // pressure spills.
    uint64_t addr = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
    asm volatile("" : "+s"(addr));
    fa_pp_tile<ACC16, BN, NS, MODE, PACKED, VNAT>(load_args(addr), tile, split);
    // Every wave has read `claimed` (and finished with the LDS ring) before
    // thread 0 claims the next tile.
    __syncthreads();
  }
}

// LDS bytes the ping-pong body needs for BN-key blocks (a ring of NS K and
// NS V or V^T blocks with padded rows).
constexpr int pp_lds_bytes(int bn, int ns, bool vnat) {
  return ns * (k_block_bytes(bn) + v_block_bytes(bn, vnat));
}

// Device entry points, one per accumulation variant. Their names contain the
// backend names of the two accumulation variants, which is how a profile
// attributes kernel time to a backend. Template parameters: BN keys per
// block, NS slots in the LDS ring, MODE (production, capture, trace, sync or split;
// each mode is a separate kernel, so the production kernels carry none of
// the debug code), PACKED (tiles of packed rows: the group's query heads
// position by position, see fa_pp_tile; also separate kernels, so the
// unpacked ones carry none of its row arithmetic), VNAT (V read in its
// natural layout through transposing LDS reads instead of the prep kernel's
// V^T). 8 waves of 64 lanes, two per SIMD.
template <int BN, int NS, int MODE, bool PACKED, bool VNAT>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
hip_fa_fp32acc_kernel(FaArgs args) {
  fa_pp_body<false, BN, NS, MODE, PACKED, VNAT>(args);
}

template <int BN, int NS, int MODE, bool PACKED, bool VNAT>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
hip_fa_fp16acc_kernel(FaArgs args) {
  fa_pp_body<true, BN, NS, MODE, PACKED, VNAT>(args);
}

// ----------------------------------------------------------------------------
// Host side: tile table, validation, launch.

typedef void (*attn_fn)(FaArgs);

struct TileConfig {
  const char* name;
  int keys;        // BN
  bool vnat;       // reads V in its natural layout (no V^T copy)
  int lds;         // dynamic LDS bytes per workgroup
  attn_fn fn[2][2][kModes];   // [packed][acc][mode]
};
constexpr int kThreads = 512;     // 8 waves
constexpr int kRows = 256;        // BM: 8 waves x 32 query rows
constexpr uint64_t kCounterBytes = 256;

#define FA_MODES(KERNEL, BN, NS, PK, VN)                                                    \
  {&KERNEL<BN, NS, MODE_RUN, PK, VN>, &KERNEL<BN, NS, MODE_CAPTURE, PK, VN>,                 \
   &KERNEL<BN, NS, MODE_TRACE, PK, VN>, &KERNEL<BN, NS, MODE_SYNC, PK, VN>,                  \
   &KERNEL<BN, NS, MODE_SPLIT, PK, VN>}
#define FA_TILE(NAME, BN, NS, VN)                                                           \
  TileConfig {                                                                              \
    NAME, BN, VN, pp_lds_bytes(BN, NS, VN), {                                               \
      {FA_MODES(hip_fa_fp32acc_kernel, BN, NS, false, VN),                                  \
       FA_MODES(hip_fa_fp16acc_kernel, BN, NS, false, VN)},                                 \
      {FA_MODES(hip_fa_fp32acc_kernel, BN, NS, true, VN),                                   \
       FA_MODES(hip_fa_fp16acc_kernel, BN, NS, true, VN)}                                   \
    }                                                                                       \
  }

// Every tile masks ragged query and key tails, applies causal masks and has
// the capture, trace and sync modes.
const TileConfig kTiles[] = {
    FA_TILE("pp_n64_r3", 64, 3, false),         // 64-key blocks, 3-slot LDS ring
    FA_TILE("pp_n64_r4", 64, 4, false),         // 64-key blocks, 4-slot LDS ring
    FA_TILE("pp_n128_r2", 128, 2, false),       // 128-key blocks, 2-slot LDS ring
    FA_TILE("pp_n128_r2_vnat", 128, 2, true),   // the same, V read in its natural layout
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);
// Automatic choice (fa_problem.kernel == 0): the 128-key tile, measured
// fastest at N = 65536 for both accumulators. Its V^T variant runs the key
// loop faster (one 16-byte LDS read per PV operand instead of two
// transposing 8-byte reads: 1.5 % at B=2 N=131072, 4-12 % on shorter or
// many-KV-head problems); its natural-V variant saves the prep kernel's pass
// over V (B * Hkv * Nk * 512 bytes of HBM traffic and a launch) and the V^T
// workspace, which matters when there is little attention work per key:
// few query rows per KV head (G * Nq, G = Hq / Hkv). Timed against each
// other (automatic split count, one session), natural V was 5 % faster at
// 1536 rows per KV head and 4-12 % slower from 3072 up; the switch sits at
// kNaturalVRows.
constexpr int kAutoVt = 3;
constexpr int kAutoNatural = 4;
constexpr int64_t kNaturalVRows = 2048;

// Query rows per KV head, or -1 for a geometry validate() rejects.
int64_t rows_per_kv_head(const fa_problem* p) {
  if (p->heads_kv <= 0 || p->heads_q <= 0 || p->seq_q <= 0 || p->heads_q % p->heads_kv) return -1;
  return p->heads_q / p->heads_kv * p->seq_q;
}

int select_tile(const fa_problem* p, const TileConfig** out) {
  int idx = p->kernel;
  if (idx == 0) {
    const int64_t rows = rows_per_kv_head(p);
    idx = rows > 0 && rows <= kNaturalVRows ? kAutoNatural : kAutoVt;
  }
  if (idx < 1 || idx > kNumTiles) return FA_ERR_KERNEL;
  *out = &kTiles[idx - 1];
  return FA_OK;
}

// Key length of the K and V buffers the attention kernel reads: Nk itself
// when the tile's key block divides it, else Nk rounded up to a whole block
// (64 or 128 keys, both whole prep groups), zero-padded by the prep kernel:
// it then writes padded copies of K and (natural-V tile) V into the
// workspace. The V^T tiles always read the prep kernel's V^T, the natural-V
// tile the caller's v (or its padded copy). The last block holds at least
// one real key.
struct KeyLayout {
  int64_t nk_pad;
  bool pad;              // ragged key tail: the kernel reads padded copies
  bool vnat;             // the tile reads V in its natural layout
  uint64_t head_bytes;   // one copy of K, V or V^T: B * Hkv * nk_pad * 128 * 2
  // Workspace: V^T (V^T tiles), the padded K, the padded V (natural-V tile),
  // then the attention kernel's tile counter in a 256-byte slot of its own.
  int copies() const { return (vnat ? 0 : 1) + (pad ? (vnat ? 2 : 1) : 0); }
  uint64_t counter_offset() const { return copies() * head_bytes; }
  uint64_t workspace_bytes() const { return counter_offset() + kCounterBytes; }
};

KeyLayout key_layout(const fa_problem* p, const TileConfig* tile) {
  KeyLayout lay;
  lay.pad = p->seq_k % tile->keys != 0;
  lay.vnat = tile->vnat;
  lay.nk_pad = lay.pad ? (p->seq_k + tile->keys - 1) / tile->keys * tile->keys : p->seq_k;
  static_assert(PAD_GROUP == 64, "key blocks of 64 and 128 are whole prep groups");
  lay.head_bytes = (uint64_t)p->batch * p->heads_kv * lay.nk_pad * HD * sizeof(_Float16);
  return lay;
}

int validate(const fa_problem* p, const TileConfig** tile) {
  if (!p) return FA_ERR_NULL;
  if (p->batch <= 0 || p->heads_q <= 0 || p->heads_kv <= 0 || p->seq_q <= 0 || p->seq_k <= 0 ||
      p->dim <= 0)
    return FA_ERR_GEOMETRY;
  if (p->heads_q % p->heads_kv) return FA_ERR_GEOMETRY;
  if (p->dim != HD) return FA_ERR_DIM;
  if (p->acc != FA_ACC_FP32 && p->acc != FA_ACC_FP16) return FA_ERR_ACC;
  if (!(p->scale > 0.f) || !isfinite(p->scale)) return FA_ERR_SCALE;
  if (p->causal != FA_CAUSAL_NONE && p->causal != FA_CAUSAL_TOP_LEFT &&
      p->causal != FA_CAUSAL_BOTTOM_RIGHT)
    return FA_ERR_CAUSAL;
  int rc = select_tile(p, tile);
  if (rc) return rc;
  // 32-bit index limits used inside the kernels (the padded key length too).
  const int64_t lim = (int64_t)1 << 30;
  if (p->seq_q >= lim || p->seq_k >= lim - 128 || p->heads_q >= lim || p->batch >= lim)
    return FA_ERR_GEOMETRY;
  const int64_t bh = p->batch * p->heads_q;
  const int64_t tiles_q = (p->seq_q + kRows - 1) / kRows;
  if (bh >= lim || bh * tiles_q >= lim || p->batch * p->heads_kv >= 65536) return FA_ERR_GEOMETRY;
  // The kernels address a head's contiguous V^T rows, or its contiguous K
  // and V rows (Nk' keys), with 32-bit byte offsets.
  if ((int64_t)HD * 2 * key_layout(p, *tile).nk_pad >= ((int64_t)1 << 31)) return FA_ERR_GEOMETRY;
  return FA_OK;
}

// FP32 values capture mode writes: 4 statistics x key blocks x B * Hq * Nq rows.
uint64_t capture_count(const fa_problem* p, const TileConfig* tile, const KeyLayout& lay) {
  return 4ull * (uint64_t)(lay.nk_pad / tile->keys) * (uint64_t)(p->batch * p->heads_q * p->seq_q);
}

// Row sequences of one attention launch (the kernel's tile rows, see
// fa_pp_tile): unpacked, B * Hq sequences of Nq query rows; packed, B * Hkv
// sequences of Nq * group rows (the group's query heads position by
// position), taken whenever that needs fewer 256-row tiles: grouped-query
// attention with fewer than 256 query rows per head, or ragged tails that
// pack tighter. Both give every row the same result bit for bit.
struct RowLayout {
  int64_t seqs;   // sequences
  int64_t rows;   // rows per sequence
  int64_t pack;   // query heads per position in a sequence: the group if packed, else 1
  int64_t tiles() const { return seqs * ((rows + kRows - 1) / kRows); }
};
RowLayout row_layout(const fa_problem* p) {
  const int64_t group = p->heads_q / p->heads_kv;
  const RowLayout plain{p->batch * p->heads_q, p->seq_q, 1};
  if (group <= 1 || p->seq_q * group >= ((int64_t)1 << 30)) return plain;
  const RowLayout packed{p->batch * p->heads_kv, p->seq_q * group, group};
  return packed.tiles() < plain.tiles() ? packed : plain;
}

// Query tiles of one attention launch (one per 256 rows of a row sequence).
uint64_t grid_size(const fa_problem* p) { return (uint64_t)row_layout(p).tiles(); }

// Split mode's partial results, after the tile counter in the workspace:
// the parts' log-sum-exp (FP32 [splits][R], R = B * Hq * Nq) from a 256-byte
// boundary, then their O (FP32 [splits][R][128]).
struct SplitLayout {
  uint64_t lpart_offset, opart_offset, end;
};
SplitLayout split_layout(const fa_problem* p, const KeyLayout& lay, int splits) {
  const uint64_t rows = (uint64_t)(p->batch * p->heads_q) * (uint64_t)p->seq_q;
  SplitLayout sl;
  sl.lpart_offset = lay.workspace_bytes();   // a multiple of 256
  sl.opart_offset = sl.lpart_offset + (splits * rows * sizeof(float) + 255) / 256 * 256;
  sl.end = sl.opart_offset + splits * rows * HD * sizeof(float);
  return sl;
}

// Largest accepted split count (fa_fwd_split's splits argument).
constexpr int kMaxSplits = 1024;
// Split counts the automatic choice considers: every count up to
// kAutoSplitMax without a mask (the model is a closed form there), these
// with a causal mask (the model sums over the tiles).
constexpr int kAutoSplitMax = 256;
constexpr int kAutoSplitsCausal[] = {2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64, 96, 128, 192, 256};

// Modelled duration of a launch whose tiles' key ranges are cut into s
// parts, in units of one key block's time on one workgroup. A work item
// costs its key blocks plus kItemOverhead (pipeline fill and drain,
// epilogue), an empty item (a causal part past the diagonal) almost nothing.
// Equal items (full attention) run in ceil(items / cus) rounds; unequal ones
// (causal) are bounded by max(total / cus, longest item), which the work
// queue, handing out the longest tiles first, comes close to. A split launch
// adds the merge kernel: it reads every part's O and lse and writes O, at
// kMergeBytesPerSecond, but no faster than one row's walk over its parts
// (four part loads in flight, kMergeLatency per four), which is what bounds
// it when the rows are few (decode shapes).
constexpr double kItemOverhead = 1.5;
constexpr double kEmptyItem = 0.1;
constexpr double kMergeBytesPerSecond = 4.0e12;
constexpr double kMergeLatency = 0.7e-6;
// fa_merge_wide_kernel takes over from fa_merge_kernel for at most this many
// rows with at least kMergeWideParts parts (one workgroup per row).
constexpr int64_t kMergeWideRows = 4096;
constexpr int kMergeWideParts = 32;
bool merge_wide(int64_t rows, int splits) { return rows <= kMergeWideRows && splits >= kMergeWideParts; }
double split_cost(const fa_problem* p, const TileConfig* tile, const KeyLayout& lay, int s, int cus) {
  const int bn = tile->keys;
  const int64_t nbt = lay.nk_pad / bn;
  const RowLayout rl = row_layout(p);
  const int64_t nbh = rl.seqs, tiles_q = (rl.rows + kRows - 1) / kRows;
  const double items = (double)(nbh * tiles_q) * s;
  double t = 0.0;
  if (p->causal == FA_CAUSAL_NONE) {
    const double per = (double)((nbt + s - 1) / s) + kItemOverhead;
    t = ceil(items / cus) * per;
  } else {
    const int64_t off = p->causal == FA_CAUSAL_BOTTOM_RIGHT ? p->seq_k - p->seq_q : 0;
    double total = 0.0, longest = 0.0;
    for (int64_t r = 0; r < tiles_q; ++r) {
      // Keys [0, kend) are seen by the tile's last row (its position + 1).
      const int64_t kend = (std::min<int64_t>((r + 1) * kRows, rl.rows) - 1) / rl.pack + 1 + off;
      const int64_t vis = kend <= 0 ? 0 : std::min<int64_t>(nbt, (kend + bn - 1) / bn);
      for (int i = 0; i < s; ++i) {
        const int64_t b0 = i * nbt / s, b1 = (i + 1) * nbt / s;
        const int64_t nb = std::max<int64_t>(0, std::min(vis, b1) - b0);
        const double cost = nb > 0 ? nb + kItemOverhead : kEmptyItem;
        total += cost * nbh;
        longest = std::max(longest, cost);
      }
    }
    t = std::max(total / cus, longest);
  }
  if (s > 1) {
    const double rows = (double)(p->batch * p->heads_q) * p->seq_q;
    const double bytes = rows * (s * (HD * 4.0 + 4.0) + HD * 2.0 + 4.0);
    const double block_seconds = bn == 128 ? 3.4e-6 : 1.8e-6;
    // A row's walk: four part loads in flight per lane, over all its parts
    // (fa_merge_kernel) or over an eighth of them (fa_merge_wide_kernel).
    const int walk = merge_wide((int64_t)rows, s) ? (s + 7) / 8 : s;
    const double merge = std::max(bytes / kMergeBytesPerSecond, ((walk + 3) / 4) * kMergeLatency);
    t += merge / block_seconds;
  }
  return t;
}

// Effective split count for a requested one: 0 picks the count with the
// shortest modelled launch (splitting only when that beats one pass over the
// keys by 10 %: tiles must leave CUs idle), n >= 1 is clamped to the tile's
// key blocks (every part then has at least one).
int resolve_splits(const fa_problem* p, const TileConfig* tile, const KeyLayout& lay,
                   int requested, int cus, int* out) {
  if (requested < 0 || requested > kMaxSplits || cus <= 0) return FA_ERR_SPLIT;
  const int64_t nbt = lay.nk_pad / tile->keys;
  int s = (int)std::min<int64_t>(requested, nbt);
  if (requested == 0) {
    s = 1;
    if (grid_size(p) < 2 * (uint64_t)cus) {
      double best = 0.9 * split_cost(p, tile, lay, 1, cus);
      auto consider = [&](int c) {
        if (c > nbt) return;
        const double t = split_cost(p, tile, lay, c, cus);
        if (t < best) {
          best = t;
          s = c;
        }
      };
      if (p->causal == FA_CAUSAL_NONE) {
        for (int c = 2; c <= kAutoSplitMax; ++c) consider(c);
      } else {
        for (int c : kAutoSplitsCausal) consider(c);
      }
    }
  }
  if ((int64_t)grid_size(p) * s >= ((int64_t)1 << 30)) return FA_ERR_GEOMETRY;
  *out = std::max(s, 1);
  return FA_OK;
}

// Strides of a contiguous [B, H, N, 128] tensor.
Strides contiguous(int64_t heads, int64_t seq) { return Strides{heads * seq * HD, seq * HD, HD}; }

Strides strides_of(const int64_t* s) { return Strides{s[0], s[1], s[2]}; }

// Caller strides must keep every 128-element row 16-byte aligned and rows
// apart (n >= 128); the K rows of one head, and its V rows if the tile reads
// them in place (natural-V tile), must span less than 2^31 bytes (32-bit
// buffer offsets) unless padded copies are read instead.
int check_strides(const fa_problem* p, const fa_strides* s, const KeyLayout& lay) {
  for (const int64_t* t : {s->q, s->k, s->v, s->o})
    for (int i = 0; i < 3; ++i) {
      if (t[i] < 0 || t[i] >= ((int64_t)1 << 40)) return FA_ERR_GEOMETRY;
      if (t[i] % 8) return FA_ERR_ALIGN;
    }
  for (const int64_t* t : {s->q, s->k, s->v, s->o})
    if (t[2] < HD) return FA_ERR_GEOMETRY;
  if (!lay.pad)
    for (const int64_t* t : {s->k, s->v})
      if ((t == s->k || lay.vnat) && (p->seq_k - 1) * t[2] * 2 + HD * 2 >= ((int64_t)1 << 31))
        return FA_ERR_GEOMETRY;
  return FA_OK;
}

// Tiles above 64 KiB of LDS need the per-kernel dynamic-LDS limit raised,
// once per kernel function and device. These flags and the per-device
// scratch addresses of fa_fwd_noalloc are the library's only host state;
// setting either twice (two threads racing on a first call) is harmless.
constexpr int kMaxDevices = 64;
std::atomic<uint8_t> g_lds_ready[kMaxDevices][kNumTiles][2][2][kModes];

int ensure_lds_limit(const TileConfig* tile, int packed, int acc, int mode) {
  if (tile->lds <= 65536) return FA_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FA_ERR_LAUNCH;
  std::atomic<uint8_t>& ready = g_lds_ready[dev][tile - kTiles][packed][acc][mode];
  if (ready.load(std::memory_order_acquire)) return FA_OK;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(tile->fn[packed][acc][mode]),
                          hipFuncAttributeMaxDynamicSharedMemorySize, tile->lds) != hipSuccess)
    return FA_ERR_LAUNCH;
  ready.store(1, std::memory_order_release);
  return FA_OK;
}

// Compute units of the current device (the persistent grid's size), looked
// up once per device.
std::atomic<int> g_cus[kMaxDevices];

int device_cus(int* cus) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FA_ERR_LAUNCH;
  int n = g_cus[dev].load(std::memory_order_acquire);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      return FA_ERR_LAUNCH;
    g_cus[dev].store(n, std::memory_order_release);
  }
  *cus = n;
  return FA_OK;
}

// The per-device state above is looked up for the current device, so a
// launch's stream must be one of that device's (the null, legacy and
// per-thread default streams always are).
int check_stream_device(void* stream) {
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!st || st == hipStreamLegacy || st == hipStreamPerThread) return FA_OK;
  int dev = 0, sdev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipStreamGetDevice(st, &sdev) != hipSuccess)
    return FA_ERR_LAUNCH;
  return sdev == dev ? FA_OK : FA_ERR_DEVICE;
}

// Optional outputs of one launch (per-row LSE, capture statistics, trace
// records) and the synchronous debug mode.
struct Extras {
  float* lse = nullptr;
  float* stats = nullptr;
  uint64_t stats_count = 0;
  uint64_t* trace = nullptr;
  uint64_t trace_count = 0;
  bool sync = false;
  bool split = false;        // fa_fwd_split: split the key range of every tile
  int splits = 0;            // requested parts (0 = automatic)
};

int launch(const fa_problem* p, const fa_strides* strides, const void* q, const void* k,
           const void* v, void* o, const Extras& ex, void* workspace, uint64_t workspace_bytes,
           void* stream) {
  const TileConfig* tile = nullptr;
  int rc = validate(p, &tile);
  if (rc) return rc;
  if (!q || !k || !v || !o) return FA_ERR_NULL;
  const KeyLayout lay = key_layout(p, tile);
  Strides qs = contiguous(p->heads_q, p->seq_q), os = qs;
  Strides ks = contiguous(p->heads_kv, p->seq_k), vs = ks;
  if (strides) {
    rc = check_strides(p, strides, lay);
    if (rc) return rc;
    qs = strides_of(strides->q);
    ks = strides_of(strides->k);
    vs = strides_of(strides->v);
    os = strides_of(strides->o);
  }
  // The automatic split count depends on the device's CU count; an explicit
  // one does not, so its errors come before any device query.
  int cus = 0;
  int splits = 1;
  if (ex.split) {
    if (ex.splits == 0) {
      rc = device_cus(&cus);
      if (rc) return rc;
    }
    rc = resolve_splits(p, tile, lay, ex.splits, cus ? cus : 1, &splits);
    if (rc) return rc;
  }
  const SplitLayout sl = split_layout(p, lay, splits);
  if (!workspace || workspace_bytes < (splits > 1 ? sl.end : lay.workspace_bytes()))
    return FA_ERR_WORKSPACE;
  for (const void* ptr : {q, k, v, (const void*)o, (const void*)workspace, (const void*)ex.lse,
                          (const void*)ex.stats, (const void*)ex.trace})
    if (reinterpret_cast<uintptr_t>(ptr) & 15) return FA_ERR_ALIGN;
  if (ex.stats && ex.stats_count < capture_count(p, tile, lay)) return FA_ERR_CAPTURE;
  if (ex.trace && ex.trace_count < grid_size(p) * TRACE_WORDS) return FA_ERR_TRACE;
  const int acc = p->acc == FA_ACC_FP16 ? 1 : 0;
  const int mode = splits > 1 ? MODE_SPLIT
                   : ex.stats ? MODE_CAPTURE
                   : ex.trace ? MODE_TRACE
                   : ex.sync  ? MODE_SYNC
                              : MODE_RUN;
  const int packed = row_layout(p).pack > 1 ? 1 : 0;
  rc = check_stream_device(stream);
  if (rc) return rc;
  rc = ensure_lds_limit(tile, packed, acc, mode);
  if (rc) return rc;
  if (!cus) {
    rc = device_cus(&cus);
    if (rc) return rc;
  }

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // Workspace: [V^T] [padded K] [padded V] counter, as the layout has them.
  _Float16* ws = static_cast<_Float16*>(workspace);
  const uint64_t head_elems = lay.head_bytes / sizeof(_Float16);
  _Float16* vt = lay.vnat ? nullptr : ws;
  _Float16* kpad = lay.pad ? ws + (lay.vnat ? 0 : head_elems) : nullptr;
  _Float16* vpad = lay.pad && lay.vnat ? kpad + head_elems : nullptr;
  int* next_tile = reinterpret_cast<int*>(static_cast<char*>(workspace) + lay.counter_offset());

  // hipLaunchKernel returns the status of this launch alone; errors left
  // pending by the caller's earlier work are neither read nor cleared.
  if (mode == MODE_SYNC) {
    // Sync mode: the workspace (V^T, padded K and V) starts as FP16 NaN, so a read
    // of any element the prep kernel does not write reaches the output.
    u32x4* ws = static_cast<u32x4*>(workspace);
    uint64_t n16 = lay.counter_offset() / 16;
    void* poison_args[] = {&ws, &n16};
    const unsigned blocks = (unsigned)std::min<uint64_t>((n16 + 255) / 256, 4096);
    if (n16 && hipLaunchKernel(reinterpret_cast<const void*>(&fa_poison_kernel), dim3(blocks),
                               dim3(256), poison_args, 0, st) != hipSuccess)
      return FA_ERR_LAUNCH;
  }
  {
    const _Float16* kk = static_cast<const _Float16*>(k);
    const _Float16* vv = static_cast<const _Float16*>(v);
    int nk_valid = (int)p->seq_k, nk_pad = (int)lay.nk_pad, heads_kv = (int)p->heads_kv;
    void* vt_args[] = {&kk, &vv, &vt, &kpad, &nk_valid, &nk_pad, &heads_kv, &ks, &vs, &next_tile};
    void* pad_args[] = {&kk, &vv, &kpad, &vpad, &nk_valid, &nk_pad, &heads_kv, &ks, &vs, &next_tile};
    const dim3 groups((unsigned)(lay.nk_pad / PAD_GROUP), (unsigned)(p->batch * p->heads_kv));
    // The natural-V tile without a key tail needs the pad kernel only for
    // the counter, which a launch of at most one work item per CU does not
    // use (fa_pp_body): then nothing runs before the attention kernel.
    const bool direct = grid_size(p) * splits <= (uint64_t)cus;
    bool ok = true;
    if (!lay.vnat)
      ok = hipLaunchKernel(reinterpret_cast<const void*>(&fa_prep_kernel), groups, dim3(256),
                           vt_args, 0, st) == hipSuccess;
    else if (lay.pad || !direct)
      ok = hipLaunchKernel(reinterpret_cast<const void*>(&fa_pad_kernel),
                           lay.pad ? groups : dim3(1, 1), dim3(256), pad_args, 0, st) == hipSuccess;
    if (!ok) return FA_ERR_LAUNCH;
  }

  FaArgs args;
  args.q = static_cast<const _Float16*>(q);
  args.k = lay.pad ? kpad : static_cast<const _Float16*>(k);
  args.v = !lay.vnat ? vt : lay.pad ? vpad : static_cast<const _Float16*>(v);
  args.o = static_cast<_Float16*>(o);
  args.lse = ex.lse;
  args.stats = ex.stats;
  args.trace = ex.trace;
  args.opart = reinterpret_cast<float*>(static_cast<char*>(workspace) + sl.opart_offset);
  args.lpart = reinterpret_cast<float*>(static_cast<char*>(workspace) + sl.lpart_offset);
  args.next_tile = next_tile;
  args.tiles = (int)grid_size(p);
  args.splits = splits;
  args.heads_q = (int)p->heads_q;
  args.group = (int)(p->heads_q / p->heads_kv);
  args.seq_q = (int)p->seq_q;
  args.seq_k = (int)lay.nk_pad;
  args.nk_valid = (int)p->seq_k;
  args.causal = p->causal != FA_CAUSAL_NONE;
  args.causal_off = p->causal == FA_CAUSAL_BOTTOM_RIGHT ? (int)(p->seq_k - p->seq_q) : 0;
  args.c = (float)((double)p->scale * LOG2E);
  args.qs = qs;
  args.os = os;
  args.ks = lay.pad ? contiguous(p->heads_kv, lay.nk_pad) : ks;
  args.vs = lay.pad || !lay.vnat ? contiguous(p->heads_kv, lay.nk_pad) : vs;
  void* attn_args[] = {&args};
  // One workgroup per CU (the LDS ring leaves room for no second one), never
  // more workgroups than work items.
  const unsigned grid = (unsigned)std::min<uint64_t>(grid_size(p) * splits, (uint64_t)cus);
  if (hipLaunchKernel(reinterpret_cast<const void*>(tile->fn[packed][acc][mode]), dim3(grid),
                      dim3(kThreads), attn_args, tile->lds, st) != hipSuccess)
    return FA_ERR_LAUNCH;
  if (splits > 1) {
    const float* opart = args.opart;
    const float* lpart = args.lpart;
    _Float16* out = args.o;
    float* lse = ex.lse;
    int nsplit = splits;
    int64_t rows = p->batch * p->heads_q * p->seq_q;
    int heads_q = (int)p->heads_q, seq_q = (int)p->seq_q;
    void* merge_args[] = {&opart, &lpart, &out, &lse, &nsplit, &rows, &heads_q, &seq_q, &os};
    const bool wide = merge_wide(rows, splits);
    const unsigned blocks =
        (unsigned)std::min<int64_t>(wide ? rows : (rows + 7) / 8, (int64_t)1 << 20);
    const void* merge_fn = wide ? reinterpret_cast<const void*>(&fa_merge_wide_kernel)
                                : reinterpret_cast<const void*>(&fa_merge_kernel);
    if (hipLaunchKernel(merge_fn, dim3(blocks), dim3(256), merge_args, 0, st) != hipSuccess)
      return FA_ERR_LAUNCH;
  }
  return FA_OK;
}

// Device address of this file's scratch array on the current device (set up
// on the first call per device, with that device current).
int scratch_address(void** out);

}  // namespace

// Workspace of fa_fwd_noalloc(): one copy per device, held from module load
// until the process ends. Host code never uses the array's name as an
// address (on the host it is only a stand-in for the symbol); it asks the
// runtime for the device address once per device and passes that on.
static __device__ __align__(256) unsigned char scratch[FA_NOALLOC_SCRATCH_BYTES];

namespace {

std::atomic<void*> g_scratch[kMaxDevices];

int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FA_ERR_LAUNCH;
  void* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (!ptr) {
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return FA_ERR_LAUNCH;
    g_scratch[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return FA_OK;
}

}  // namespace

extern "C" {

int fa_fwd_noalloc(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
                   void* stream) {
  uint64_t need = 0;
  int rc = fa_fwd_workspace_bytes(p, &need);
  if (rc) return rc;
  if (need > FA_NOALLOC_SCRATCH_BYTES) return FA_ERR_SCRATCH;
  if (!q || !k || !v || !o) return FA_ERR_NULL;
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc) return rc;
  return launch(p, nullptr, q, k, v, o, Extras{}, ws, FA_NOALLOC_SCRATCH_BYTES, stream);
}

int fa_fwd_workspace_bytes(const fa_problem* p, uint64_t* bytes) {
  if (!bytes) return FA_ERR_NULL;
  const TileConfig* tile = nullptr;
  int rc = validate(p, &tile);
  if (rc) return rc;
  const KeyLayout lay = key_layout(p, tile);
  *bytes = lay.workspace_bytes();
  return FA_OK;
}

int fa_fwd_tile(const fa_problem* p, int32_t* rows, int32_t* keys) {
  if (!p || !rows || !keys) return FA_ERR_NULL;
  const TileConfig* tile = nullptr;
  int rc = select_tile(p, &tile);
  if (rc) return rc;
  *rows = 1;          // every tile masks ragged query and key tails
  *keys = 1;
  return FA_OK;
}

int fa_fwd_select(const fa_problem* p, int32_t* kernel) {
  if (!p || !kernel) return FA_ERR_NULL;
  const TileConfig* tile = nullptr;
  int rc = select_tile(p, &tile);
  if (rc) return rc;
  *kernel = (int32_t)(tile - kTiles) + 1;
  return FA_OK;
}

int fa_fwd(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
           void* workspace, uint64_t workspace_bytes, void* stream) {
  return launch(p, nullptr, q, k, v, o, Extras{}, workspace, workspace_bytes, stream);
}

int fa_fwd_lse(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
               float* lse, void* workspace, uint64_t workspace_bytes, void* stream) {
  Extras ex;
  ex.lse = lse;
  return launch(p, nullptr, q, k, v, o, ex, workspace, workspace_bytes, stream);
}

int fa_fwd_strided(const fa_problem* p, const fa_strides* strides, const void* q, const void* k,
                   const void* v, void* o, float* lse, void* workspace, uint64_t workspace_bytes,
                   void* stream) {
  if (!strides) return FA_ERR_NULL;
  Extras ex;
  ex.lse = lse;
  return launch(p, strides, q, k, v, o, ex, workspace, workspace_bytes, stream);
}

int fa_fwd_capture_count(const fa_problem* p, uint64_t* count, int32_t* block_keys) {
  if (!count || !block_keys) return FA_ERR_NULL;
  const TileConfig* tile = nullptr;
  int rc = validate(p, &tile);
  if (rc) return rc;
  *count = capture_count(p, tile, key_layout(p, tile));
  *block_keys = tile->keys;
  return FA_OK;
}

int fa_fwd_capture(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
                   float* lse, float* stats, uint64_t stats_count, void* workspace,
                   uint64_t workspace_bytes, void* stream) {
  if (!stats) return FA_ERR_NULL;
  Extras ex;
  ex.lse = lse;
  ex.stats = stats;
  ex.stats_count = stats_count;
  return launch(p, nullptr, q, k, v, o, ex, workspace, workspace_bytes, stream);
}

int fa_fwd_trace_count(const fa_problem* p, uint64_t* count) {
  if (!count) return FA_ERR_NULL;
  const TileConfig* tile = nullptr;
  int rc = validate(p, &tile);
  if (rc) return rc;
  *count = grid_size(p) * TRACE_WORDS;
  return FA_OK;
}

int fa_fwd_trace(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
                 uint64_t* trace, uint64_t trace_count, void* workspace, uint64_t workspace_bytes,
                 void* stream) {
  if (!trace) return FA_ERR_NULL;
  Extras ex;
  ex.trace = trace;
  ex.trace_count = trace_count;
  return launch(p, nullptr, q, k, v, o, ex, workspace, workspace_bytes, stream);
}

int fa_fwd_sync(const fa_problem* p, const void* q, const void* k, const void* v, void* o,
                float* lse, void* workspace, uint64_t workspace_bytes, void* stream) {
  Extras ex;
  ex.lse = lse;
  ex.sync = true;
  return launch(p, nullptr, q, k, v, o, ex, workspace, workspace_bytes, stream);
}

int fa_fwd_split_count(const fa_problem* p, int32_t splits, int32_t cus, int32_t* effective) {
  if (!effective) return FA_ERR_NULL;
  const TileConfig* tile = nullptr;
  int rc = validate(p, &tile);
  if (rc) return rc;
  if (cus < 0) return FA_ERR_SPLIT;
  int n = cus;
  if (n == 0) {
    rc = device_cus(&n);
    if (rc) return rc;
  }
  int s = 0;
  rc = resolve_splits(p, tile, key_layout(p, tile), splits, n, &s);
  if (rc) return rc;
  *effective = s;
  return FA_OK;
}

int fa_fwd_split_workspace_bytes(const fa_problem* p, int32_t splits, uint64_t* bytes) {
  if (!bytes) return FA_ERR_NULL;
  const TileConfig* tile = nullptr;
  int rc = validate(p, &tile);
  if (rc) return rc;
  const KeyLayout lay = key_layout(p, tile);
  int cus = 1;   // an explicit count does not depend on the device
  if (splits == 0) {
    rc = device_cus(&cus);
    if (rc) return rc;
  }
  int s = 0;
  rc = resolve_splits(p, tile, lay, splits, cus, &s);
  if (rc) return rc;
  *bytes = s > 1 ? split_layout(p, lay, s).end : lay.workspace_bytes();
  return FA_OK;
}

int fa_fwd_split(const fa_problem* p, int32_t splits, const fa_strides* strides, const void* q,
                 const void* k, const void* v, void* o, float* lse, void* workspace,
                 uint64_t workspace_bytes, void* stream) {
  Extras ex;
  ex.lse = lse;
  ex.split = true;
  ex.splits = splits;
  return launch(p, strides, q, k, v, o, ex, workspace, workspace_bytes, stream);
}

int fa_kernel_count(void) { return kNumTiles; }

const char* fa_kernel_name(int32_t kernel) {
  if (kernel < 1 || kernel > kNumTiles) return nullptr;
  return kTiles[kernel - 1].name;
}

const char* fa_strerror(int status) {
  switch (status) {
    case FA_OK: return "ok";
    case FA_ERR_NULL: return "required pointer is NULL";
    case FA_ERR_GEOMETRY: return "invalid attention geometry";
    case FA_ERR_DIM: return "head dimension must be 128";
    case FA_ERR_TAIL: return "unsupported query/key tail (no longer returned: every tile masks tails)";
    case FA_ERR_ALIGN: return "tensor pointer not 16-byte aligned";
    case FA_ERR_WORKSPACE: return "workspace missing or too small";
    case FA_ERR_ACC: return "unknown accumulation variant";
    case FA_ERR_SCALE: return "scale must be finite and positive";
    case FA_ERR_KERNEL: return "unknown kernel selector";
    case FA_ERR_LAUNCH: return "HIP kernel launch failed";
    case FA_ERR_CAPTURE: return "capture needs a stats buffer of fa_fwd_capture_count() floats";
    case FA_ERR_CAUSAL: return "unknown causal mode";
    case FA_ERR_TRACE: return "trace needs a buffer of fa_fwd_trace_count() 64-bit words";
    case FA_ERR_SCRATCH: return "problem needs more workspace than fa_fwd_noalloc's scratch (FA_NOALLOC_SCRATCH_BYTES)";
    case FA_ERR_SPLIT: return "split count outside 0..1024 (or a negative CU count)";
    case FA_ERR_DEVICE: return "stream belongs to another device than the current one";
    default: return "unknown status";
  }
}

}  // extern "C"
