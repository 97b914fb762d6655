// Sustained dense FP16 MFMA rate of the board: a measurement kernel, not part
// of the attention library. Modes 0-4 share the attention kernel's launch
// shape (8 waves of 64 lanes per workgroup, two waves per SIMD), modes 5-6
// run one wave per SIMD; all use its matrix instruction
// (v_mfma_f32_32x32x16_f16), and
// does nothing but issue those instructions for a fixed number of
// iterations, so its rate is what the matrix cores sustain on this board
// under its power limit when nothing else runs beside them.
//
//   MODE 0  operands in registers: the matrix pipe alone.
//   MODE 1  each MFMA's A operand is first read from LDS (one ds_read_b128
//           per lane, four reads in flight), as a GEMM or the attention
//           kernel's MFMA step feeds the pipe.
//   MODE 2  MODE 1 plus, after every MFMA, the attention kernel's softmax
//           work per MFMA: one v_exp_f32 and three other FP32 VALU
//           operations (the forward issues about 240 VALU instructions, 64
//           of them exponentials, per 64 MFMAs), on registers independent
//           of the MFMAs, so nothing waits on a result: the rate of a
//           pipeline with the forward's operand traffic and instruction mix
//           but without its data dependencies and barriers.
//   MODE 3  each A operand read from LDS feeds two MFMAs (with different B
//           operands): the LDS traffic a wave with 64 query rows would
//           have, half of the attention kernel's.
//   MODE 4  both operands of every MFMA read from LDS (2 KiB per MFMA and
//           wave, twice the attention kernel's traffic): how close LDS
//           bandwidth comes to limiting the matrix pipe.
//   MODE 5  one wave per SIMD (4 waves per workgroup, up to 512 registers
//           per lane), each A operand read from LDS feeding two MFMAs, eight
//           reads in flight: the issue rate of the single-wave layout a tile
//           of 64 query rows per wave would need.
//   MODE 6  mode 5 plus, after every MFMA, the same VALU mix as mode 2 in
//           the same wave: a 64-row-per-wave softmax overlapped with its own
//           matrix work, without dependencies.
//
// Modes 7-12 are the attention kernel's skeleton (pingpong_body): its
// registers, its MFMA step (64 MFMAs, QK into four S tiles interleaved with
// PV into four O tiles, the A operand read from LDS four MFMAs ahead) and
// its ping-pong schedule (waves w and w + 4 share a SIMD; group 0 runs an
// MFMA step while group 1 runs a VALU step, then they swap, with a
// workgroup barrier between phases), with the softmax's VALU step reduced
// or replaced so that each part's cost shows. The VALU step reads the S
// tiles the wave's own MFMA step wrote, and its P feeds the next PV
// products, as in the forward; what the skeleton leaves out is the K/V
// staging (no loads into LDS) and the O rescale.
//   MODE 7  no VALU step: MFMA steps, LDS operand reads and barriers only.
//   MODE 8  the softmax VALU step with the row sum by v_dot2c_f32_f16
//           (one FP16 dot product per pair of P values).
//   MODE 9  the softmax VALU step as the attention kernel runs it: row max
//           (v_maximum3 tree), P = exp2(s c - m c) (FMA + v_exp_f32), FP16
//           packing (v_cvt_pk_f16_f32), row sum by v_fma_mix_f32.
//   MODE 10 mode 9 without the exponentials.
//   MODE 11 mode 9 without the FP16 packing and the row sum.
//   MODE 12 mode 9 without the row sum.
//
// Every mode allocates the 16 KiB LDS operand buffer, mode 0 included (its
// final sum reads one element of it, so the compiler keeps the buffer): the
// attention kernel allocates LDS, and a mode-0 kernel that allocated none was
// measured 8 % slower at a 13 % higher clock (1502-1509 against 1634-1640
// TFLOP/s, 1828-1850 against 1614-1622 MHz, same session), the signature of
// SIMDs left idle part of the time rather than of the matrix pipe's rate.
//
// Operands are FP16 values supplied by the caller (random normal data, so the
// datapath toggles as it does on real inputs). Every wave keeps four
// independent accumulators (a dependent MFMA reuses its accumulator four
// instructions later) and writes their sum at the end, so no MFMA is dead.
// With a trace buffer, thread 0 of every workgroup records s_memrealtime and
// s_memtime at entry and after the loop (words 1-4 of an 8-word record, the
// attention kernel's trace layout), from which the running shader clock
// follows.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 512;         // two waves per SIMD (modes 0-4, 7-12)
constexpr int kThreadsSingle = 256;   // one wave per SIMD (modes 5, 6)
constexpr int kPingPongMfma = 64;     // MFMAs per MFMA step of the skeleton (modes 7-12)
constexpr int kOperandHalves = 8192;   // 16 KiB of FP16 operands
constexpr int kTraceWords = 8;
constexpr int kMfmaPerIter = 16;

__device__ __forceinline__ f32x16 mfma32(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int MODE, int NT>
__device__ __forceinline__ void ceiling_body(const _Float16* __restrict__ operands,
                                             float* __restrict__ out, uint64_t* __restrict__ trace,
                                             int iters) {
  const uint64_t real0 = __builtin_amdgcn_s_memrealtime();
  const uint64_t clk0 = __builtin_amdgcn_s_memtime();
  __shared__ __attribute__((aligned(16))) _Float16 lds[kOperandHalves];
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < kOperandHalves / 8; i += NT)
    reinterpret_cast<h8*>(lds)[i] = reinterpret_cast<const h8*>(operands)[i];
  h8 a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = reinterpret_cast<const h8*>(operands)[(j * 64 + lane) & (kOperandHalves / 8 - 1)];
    b[j] = reinterpret_cast<const h8*>(operands)[(256 + j * 64 + lane) & (kOperandHalves / 8 - 1)];
  }
  // MODE 2's VALU operands: bounded values (2^w / 2 maps [-1, 1] into
  // [0.25, 1]; the fused multiply-adds contract towards zero).
  float w[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) w[j] = (float)operands[(lane * 16 + j) & (kOperandHalves - 1)] * 0.01f;
  __syncthreads();
  f32x16 acc[4] = {};
  // LDS operand address of MFMA n of an iteration: 16 B per lane, 1 KiB per
  // MFMA, cycling through the 16 KiB buffer (distinct lanes, distinct banks).
  const char* base = reinterpret_cast<const char*>(lds) + lane * 16;
  // Modes 5 and 6: the eight operand fragments of the first iteration, read
  // in the order the loop reads them, so the compiler's wait counts stay the
  // same from one iteration to the next and no iteration drains the reads.
  h8 fr8[kMfmaPerIter / 2];
  if constexpr (MODE == 5 || MODE == 6) {
#pragma unroll
    for (int f = 0; f < kMfmaPerIter / 2; ++f) {
      fr8[f] = *reinterpret_cast<const h8*>(base + f * 1024);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  for (int it = 0; it < iters; ++it) {
    if constexpr (MODE == 0) {
#pragma unroll
      for (int n = 0; n < kMfmaPerIter; ++n) acc[n & 3] = mfma32(a[n >> 2], b[n & 3], acc[n & 3]);
    } else if constexpr (MODE == 5 || MODE == 6) {
      // Eight reads in flight across iterations: operand f of an iteration
      // is read while the previous iteration's operand f feeds its MFMAs
      // (the addresses repeat every iteration), so a single wave never
      // waits for LDS at an iteration boundary.
#pragma unroll
      for (int f = 0; f < kMfmaPerIter / 2; ++f) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int n = 2 * f + u;
          acc[n & 3] = mfma32(fr8[f], b[u], acc[n & 3]);
          if constexpr (MODE == 6) {
            w[n] = __builtin_amdgcn_exp2f(w[n]) * 0.5f;
            w[(n + 5) & 15] = __builtin_fmaf(w[(n + 5) & 15], 0.999f, -0.001f);
            w[(n + 11) & 15] = __builtin_fmaf(w[(n + 11) & 15], 0.999f, -0.001f);
          }
        }
        // Read after the fragment's last use, into the same registers.
        fr8[f] = *reinterpret_cast<const h8*>(base + f * 1024);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (MODE == 4) {
      h8 fa[4], fb[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        fa[f] = *reinterpret_cast<const h8*>(base + f * 1024);
        fb[f] = *reinterpret_cast<const h8*>(base + (8 + f) * 1024);
      }
#pragma unroll
      for (int n = 0; n < kMfmaPerIter; ++n) {
        const h8 x = fa[n & 3], y = fb[n & 3];
        if (n + 4 < kMfmaPerIter) {
          fa[n & 3] = *reinterpret_cast<const h8*>(base + ((n + 4) & 7) * 1024);
          fb[n & 3] = *reinterpret_cast<const h8*>(base + (8 + ((n + 4) & 7)) * 1024);
        }
        acc[n & 3] = mfma32(x, y, acc[n & 3]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (MODE == 3) {
      h8 fr[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) fr[f] = *reinterpret_cast<const h8*>(base + f * 1024);
#pragma unroll
      for (int f = 0; f < kMfmaPerIter / 2; ++f) {
        const h8 x = fr[f & 3];
        if (f + 4 < kMfmaPerIter / 2) fr[f & 3] = *reinterpret_cast<const h8*>(base + (f + 4) * 1024);
        acc[(2 * f) & 3] = mfma32(x, b[0], acc[(2 * f) & 3]);
        acc[(2 * f + 1) & 3] = mfma32(x, b[1], acc[(2 * f + 1) & 3]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      h8 fr[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) fr[n] = *reinterpret_cast<const h8*>(base + n * 1024);
#pragma unroll
      for (int n = 0; n < kMfmaPerIter; ++n) {
        const h8 x = fr[n & 3];
        if (n + 4 < kMfmaPerIter) fr[n & 3] = *reinterpret_cast<const h8*>(base + (n + 4) * 1024);
        acc[n & 3] = mfma32(x, b[n & 3], acc[n & 3]);
        if constexpr (MODE == 2) {
          w[n] = __builtin_amdgcn_exp2f(w[n]) * 0.5f;
          w[(n + 5) & 15] = __builtin_fmaf(w[(n + 5) & 15], 0.999f, -0.001f);
          w[(n + 11) & 15] = __builtin_fmaf(w[(n + 11) & 15], 0.999f, -0.001f);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  float sum = (float)lds[tid & 7];   // keeps the LDS buffer allocated in every mode
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += acc[j][r];
  if constexpr (MODE == 2 || MODE == 6) {
#pragma unroll
    for (int j = 0; j < 16; ++j) sum += w[j];
  }
  out[(size_t)blockIdx.x * NT + tid] = sum;
  if (trace) {
    const uint64_t real1 = __builtin_amdgcn_s_memrealtime();
    const uint64_t clk1 = __builtin_amdgcn_s_memtime();
    if (tid == 0) {
      uint64_t* rec = trace + (size_t)blockIdx.x * kTraceWords;
      rec[0] = 0;
      rec[1] = real0;
      rec[2] = real1;
      rec[3] = clk0;
      rec[4] = clk1;
      rec[5] = blockIdx.x;
      rec[6] = (uint64_t)iters;
      rec[7] = kMfmaPerIter;
    }
  }
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float smax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// acc + the FP16 value in half HI of x (the attention kernel's row-sum add).
template <int HI>
__device__ __forceinline__ float add_f16(float acc, h2 x) {
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(x));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(x));
  return acc;
}

__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Modes 7-12: the attention kernel's ping-pong skeleton (see the header).
// Each iteration is one MFMA step and one VALU step per wave, two phases.
template <int MODE>
__device__ __forceinline__ void pingpong_body(const _Float16* __restrict__ operands,
                                              float* __restrict__ out, uint64_t* __restrict__ trace,
                                              int iters) {
  constexpr bool SOFTMAX = MODE != 7, EXP = MODE != 10, PACK = MODE != 11;
  constexpr bool ROWSUM = MODE != 11 && MODE != 12, DOT2 = MODE == 8;
  const uint64_t real0 = __builtin_amdgcn_s_memrealtime();
  const uint64_t clk0 = __builtin_amdgcn_s_memtime();
  __shared__ __attribute__((aligned(16))) _Float16 lds[kOperandHalves];
  const int tid = threadIdx.x, lane = tid & 63;
  const int grp = __builtin_amdgcn_readfirstlane(tid >> 6) >> 2;
  for (int i = tid; i < kOperandHalves / 8; i += kThreads)
    reinterpret_cast<h8*>(lds)[i] = reinterpret_cast<const h8*>(operands)[i];
  // Q fragments (B operands of the QK products) and the first P.
  h8 qf[8], p[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    qf[j] = reinterpret_cast<const h8*>(operands)[(256 + j * 64 + lane) & (kOperandHalves / 8 - 1)];
    p[j] = reinterpret_cast<const h8*>(operands)[(j * 64 + lane) & (kOperandHalves / 8 - 1)];
  }
  const float c = 0.127f;                  // a softmax scale: P = 2^(s c - m c) <= 1
  const h2 ones = {(_Float16)1.f, (_Float16)1.f};
  float lsum = 0.f;
  __syncthreads();
  f32x16 s[4] = {}, o[4] = {};
  const char* base = reinterpret_cast<const char*>(lds) + lane * 16;
  auto ld = [&](int i) -> h8 { return *reinterpret_cast<const h8*>(base + (i & 15) * 1024); };
  auto mfma_step = [&]() {
    h8 fr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) fr[i] = ld(i);
#pragma unroll
    for (int i = 0; i < kPingPongMfma; ++i) {
      const int n = i >> 1;
      // Each S tile's first product starts from zero, as in the forward.
      if ((i & 1) == 0) s[n & 3] = mfma32(fr[i & 3], qf[n >> 2], n < 4 ? f32x16{} : s[n & 3]);
      else o[n & 3] = mfma32(fr[i & 3], p[n >> 2], o[n & 3]);
      if (i + 4 < kPingPongMfma) fr[i & 3] = ld(i + 4);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto valu_step = [&]() {
    if constexpr (!SOFTMAX) {
#pragma unroll
      for (int t = 0; t < 4; ++t) asm volatile("" ::"v"(s[t]));
      return;
    }
    float mv[64];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mv[16 * t + r] = s[t][r];
#pragma unroll
    for (int n = 64; n > 1; n = (n + 2) / 3) {
#pragma unroll
      for (int i = 0; 3 * i < n; ++i) {
        float x = mv[3 * i];
        if (3 * i + 1 < n) x = smax(x, mv[3 * i + 1]);
        if (3 * i + 2 < n) x = smax(x, mv[3 * i + 2]);
        mv[i] = x;
      }
    }
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mv[0]), __float_as_uint(mv[0]), false, false);
    const float mc = smax(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * c;
    float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        h8 frag;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float p0 = __builtin_fmaf(s[t][8 * g2 + e], c, -mc);
          float p1 = __builtin_fmaf(s[t][8 * g2 + e + 1], c, -mc);
          if constexpr (EXP) {
            p0 = __builtin_amdgcn_exp2f(p0);
            p1 = __builtin_amdgcn_exp2f(p1);
          }
          if constexpr (PACK) {
            const h2 pr = {(_Float16)p0, (_Float16)p1};
            frag[e] = pr[0];
            frag[e + 1] = pr[1];
            if constexpr (DOT2) {
              ls[e >> 1] = __builtin_amdgcn_fdot2(pr, ones, ls[e >> 1], false);
            } else if constexpr (ROWSUM) {
              ls[e >> 1] = add_f16<0>(ls[e >> 1], pr);
              ls[(e >> 1) ^ 2] = add_f16<1>(ls[(e >> 1) ^ 2], pr);
            }
          } else {
            asm volatile("" ::"v"(p0), "v"(p1));
          }
        }
        if constexpr (PACK) p[2 * t + g2] = frag;
      }
    lsum += (ls[0] + ls[1]) + (ls[2] + ls[3]);
  };
  // Both groups pass 2 * iters barriers.
  if (grp == 0) {
    for (int it = 0; it < iters; ++it) {
      mfma_step();
      phase_barrier();
      valu_step();
      phase_barrier();
    }
  } else {
    for (int it = 0; it < iters; ++it) {
      valu_step();
      phase_barrier();
      mfma_step();
      phase_barrier();
    }
  }
  float sum = lsum + (float)lds[tid & 7];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += o[j][r] + s[j][r];
  out[(size_t)blockIdx.x * kThreads + tid] = sum;
  if (trace) {
    const uint64_t real1 = __builtin_amdgcn_s_memrealtime();
    const uint64_t clk1 = __builtin_amdgcn_s_memtime();
    if (tid == 0) {
      uint64_t* rec = trace + (size_t)blockIdx.x * kTraceWords;
      rec[0] = 0;
      rec[1] = real0;
      rec[2] = real1;
      rec[3] = clk0;
      rec[4] = clk1;
      rec[5] = blockIdx.x;
      rec[6] = (uint64_t)iters;
      rec[7] = kPingPongMfma;
    }
  }
}

template <int MODE>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
fa_pingpong_ceiling_kernel(const _Float16* __restrict__ operands, float* __restrict__ out,
                           uint64_t* __restrict__ trace, int iters) {
  pingpong_body<MODE>(operands, out, trace, iters);
}

template <int MODE>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
fa_mfma_ceiling_kernel(const _Float16* __restrict__ operands, float* __restrict__ out,
                       uint64_t* __restrict__ trace, int iters) {
  ceiling_body<MODE, kThreads>(operands, out, trace, iters);
}

template <int MODE>
__global__ void __launch_bounds__(kThreadsSingle) __attribute__((amdgpu_waves_per_eu(1, 1)))
fa_mfma_ceiling_single_kernel(const _Float16* __restrict__ operands, float* __restrict__ out,
                              uint64_t* __restrict__ trace, int iters) {
  ceiling_body<MODE, kThreadsSingle>(operands, out, trace, iters);
}

constexpr int kModes = 13;
int threads_of(int mode) { return mode == 5 || mode == 6 ? kThreadsSingle : kThreads; }
// MFMAs one wave issues per iteration.
int mfma_per_iter(int mode) { return mode >= 7 ? kPingPongMfma : kMfmaPerIter; }

}  // namespace

extern "C" {

// FP16 FLOPs one workgroup performs in modes 0-4: 8 waves x iters x 16
// MFMAs x 32x32x16x2.
uint64_t fa_ceiling_flops_per_workgroup(int iters) {
  return (uint64_t)(kThreads / 64) * (uint64_t)iters * kMfmaPerIter * 32 * 32 * 16 * 2;
}

// Threads per workgroup of a mode (512, or 256 for the one-wave-per-SIMD
// modes 5 and 6; 0 for an unknown mode) and the FP16 FLOPs one workgroup
// performs in it (16 MFMAs per wave and iteration in modes 0-6, one
// 64-MFMA step in modes 7-12).
int fa_ceiling_threads(int mode) { return mode < 0 || mode >= kModes ? 0 : threads_of(mode); }
uint64_t fa_ceiling_flops(int mode, int iters) {
  if (fa_ceiling_threads(mode) == 0) return 0;
  return (uint64_t)(fa_ceiling_threads(mode) / 64) * (uint64_t)iters * mfma_per_iter(mode) * 32 *
         32 * 16 * 2;
}

// Launch the ceiling kernel: mode 0 (register operands), 1 (LDS-fed A
// operand), 2 (LDS-fed A operand and the softmax's VALU mix), 3 (one LDS
// read per two MFMAs), 4 (both operands from LDS), 5 (one wave per SIMD,
// one LDS read per two MFMAs), 6 (mode 5 and the VALU mix) or 7-12 (the
// attention kernel's ping-pong skeleton with its softmax step in part or
// whole, see the header); operands = 8192 FP16 values
// (16-byte aligned), out = workgroups x fa_ceiling_threads(mode) floats,
// trace = workgroups x 8 words or NULL. Returns 0, or 1 for bad arguments,
// 2 when the launch is rejected.
int fa_ceiling_mfma(int mode, int workgroups, int iters, const void* operands, float* out,
                    uint64_t* trace, void* stream) {
  if (mode < 0 || mode >= kModes || workgroups <= 0 || iters <= 0 || !operands || !out) return 1;
  if ((reinterpret_cast<uintptr_t>(operands) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(trace)) & 15)
    return 1;
  const _Float16* ops = static_cast<const _Float16*>(operands);
  void* args[] = {&ops, &out, &trace, &iters};
  const void* fns[] = {reinterpret_cast<const void*>(&fa_mfma_ceiling_kernel<0>),
                       reinterpret_cast<const void*>(&fa_mfma_ceiling_kernel<1>),
                       reinterpret_cast<const void*>(&fa_mfma_ceiling_kernel<2>),
                       reinterpret_cast<const void*>(&fa_mfma_ceiling_kernel<3>),
                       reinterpret_cast<const void*>(&fa_mfma_ceiling_kernel<4>),
                       reinterpret_cast<const void*>(&fa_mfma_ceiling_single_kernel<5>),
                       reinterpret_cast<const void*>(&fa_mfma_ceiling_single_kernel<6>),
                       reinterpret_cast<const void*>(&fa_pingpong_ceiling_kernel<7>),
                       reinterpret_cast<const void*>(&fa_pingpong_ceiling_kernel<8>),
                       reinterpret_cast<const void*>(&fa_pingpong_ceiling_kernel<9>),
                       reinterpret_cast<const void*>(&fa_pingpong_ceiling_kernel<10>),
                       reinterpret_cast<const void*>(&fa_pingpong_ceiling_kernel<11>),
                       reinterpret_cast<const void*>(&fa_pingpong_ceiling_kernel<12>)};
  static_assert(sizeof(fns) / sizeof(fns[0]) == kModes, "one kernel per mode");
  const void* fn = fns[mode];
  return hipLaunchKernel(fn, dim3((unsigned)workgroups), dim3((unsigned)threads_of(mode)), args,
                         0, static_cast<hipStream_t>(stream)) == hipSuccess ? 0 : 2;
}

}  // extern "C"
