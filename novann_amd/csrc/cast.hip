// Cast, amax and scale kernels (HBM-bound streaming) for gfx950.
//
// Layout: each thread moves a few "units" (4; 2 for 16 -> 32-bit); a unit is EPL
// consecutive elements, sized so that the wider side of the cast is one
// 16-byte access per lane (the narrower side is 2 to 8 bytes: fp32 <-> fp4
// moves 16 bytes against 2).  Unit u of a block sits at (block * units_per_thread + j) *
// blockDim + tid, so every load and store instruction of a wave covers one
// contiguous span (fully coalesced).  All loads of a thread are issued before
// any conversion, to keep several 16-byte requests in flight per lane.  The
// ragged tail (n % EPL elements) is converted by one thread of the last block.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "novaq_convert.h"
#include "novaq_internal.h"

namespace novaq {

constexpr int kCastThreads = 256;
constexpr int kUnitsPerThread = 4;

template <int ST, int DT>
struct CastShape {
  static constexpr int bmax = dtype_bits(ST) > dtype_bits(DT) ? dtype_bits(ST) : dtype_bits(DT);
  static constexpr int epl = 128 / bmax;               // elements per unit
  static constexpr int src_bits = epl * dtype_bits(ST);  // bits per unit, 16 .. 128
  static constexpr int dst_bits = epl * dtype_bits(DT);
  static constexpr int src_words = (src_bits + 31) / 32;  // 32-bit words holding a unit
  static constexpr int dst_words = (dst_bits + 31) / 32;
  // units per thread: 1 for 16 -> 32-bit widening (four times the
  // workgroups: bf16 -> fp32 on 2^28 elements 271 us at 4 units, 255 at 2,
  // 252 at 1), 2 for 32 -> 16-bit narrowing (fp32 -> bf16 6.29 -> 6.63 TB/s
  // back to back); 8 units and the 8 / 4 -> 32-bit casts at 2 units measured
  // slower
  static constexpr int upt =
      dtype_bits(ST) == 16 && dtype_bits(DT) == 32 ? kUnitsPerThread / 4
      : dtype_bits(ST) == 32 && dtype_bits(DT) == 16 ? kUnitsPerThread / 2 : kUnitsPerThread;
};

template <int N>
struct Words {
  uint32_t w[N];
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Element i of a unit held as 32-bit words, for element width BITS.
template <int BITS, int N>
__device__ __forceinline__ uint32_t get_elem(const Words<N>& v, int i) {
  constexpr int per = 32 / BITS;
  constexpr uint32_t mask = (uint32_t)((1ull << BITS) - 1ull);
  return (v.w[i / per] >> ((i % per) * BITS)) & mask;
}

template <int BITS, int N>
__device__ __forceinline__ void put_elem(Words<N>& v, int i, uint32_t c) {
  constexpr int per = 32 / BITS;
  constexpr uint32_t mask = (uint32_t)((1ull << BITS) - 1ull);
  if ((i % per) == 0) v.w[i / per] = c & mask;
  else v.w[i / per] |= (c & mask) << ((i % per) * BITS);
}

// One unit of BITS bits (16 .. 128) at byte address p.
template <int BITS, int N = (BITS + 31) / 32>
__device__ __forceinline__ Words<N> load_words(const uint8_t* __restrict__ bp) {
  Words<N> v;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(bp);
  if constexpr (BITS == 16) {
    v.w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(bp));
  } else if constexpr (N % 4 == 0) {
#pragma unroll
    for (int k = 0; k < N / 4; ++k) {
      u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + k);
      v.w[4 * k] = q.x; v.w[4 * k + 1] = q.y; v.w[4 * k + 2] = q.z; v.w[4 * k + 3] = q.w;
    }
  } else if constexpr (N == 2) {
    u32x2 q = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    v.w[0] = q.x; v.w[1] = q.y;
  } else {
    static_assert(N == 1, "unit width");
    v.w[0] = __builtin_nontemporal_load(p);
  }
  return v;
}

template <int BITS, int N = (BITS + 31) / 32>
__device__ __forceinline__ void store_words(uint8_t* __restrict__ bp, const Words<N>& v) {
  uint32_t* p = reinterpret_cast<uint32_t*>(bp);
  if constexpr (BITS == 16) {
    __builtin_nontemporal_store((uint16_t)v.w[0], reinterpret_cast<uint16_t*>(bp));
  } else if constexpr (N % 4 == 0) {
#pragma unroll
    for (int k = 0; k < N / 4; ++k) {
      u32x4 q = {v.w[4 * k], v.w[4 * k + 1], v.w[4 * k + 2], v.w[4 * k + 3]};
      __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(p) + k);
    }
  } else if constexpr (N == 2) {
    u32x2 q = {v.w[0], v.w[1]};
    __builtin_nontemporal_store(q, reinterpret_cast<u32x2*>(p));
  } else {
    static_assert(N == 1, "unit width");
    __builtin_nontemporal_store(v.w[0], p);
  }
}

// Scalar element access for the ragged tail.
template <int DT>
__device__ __forceinline__ uint32_t load_scalar(const uint8_t* p, int64_t i) {
  if constexpr (dtype_bits(DT) == 32) return reinterpret_cast<const uint32_t*>(p)[i];
  else if constexpr (dtype_bits(DT) == 16) return reinterpret_cast<const uint16_t*>(p)[i];
  else if constexpr (dtype_bits(DT) == 8) return p[i];
  else return (p[i >> 1] >> ((i & 1) * 4)) & 0xFu;
}

// Scale setup: mode 0 none, 1 *scale holds s, 2 *scale holds amax (s derived,
// written to scale_out by block 0).
template <int DT>
__device__ __forceinline__ float scale_from_amax_dev(float amax) {
  return (amax > 0.0f && amax <= 3.40282347e38f) ? amax / fmt_max(DT) : 1.0f;
}

template <int ST, int DT, int SMODE>
__global__ __launch_bounds__(kCastThreads) void cast_kernel(
    const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t n,
    const float* __restrict__ scale, float* __restrict__ scale_out) {
  using Sh = CastShape<ST, DT>;
  constexpr int EPL = Sh::epl;
  constexpr bool SCALED = SMODE != 0;
  float s = 1.0f, inv_s = 1.0f;
  if constexpr (SMODE == 1) {
    s = *scale;
    inv_s = 1.0f / s;
  } else if constexpr (SMODE == 2) {
    s = scale_from_amax_dev<is_quant(DT) ? DT : ST>(*scale);
    inv_s = 1.0f / s;
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = s;
  }
  const int64_t units = n / EPL;
  const int64_t base = (int64_t)blockIdx.x * Sh::upt * kCastThreads + threadIdx.x;

  Words<Sh::src_words> in[Sh::upt];
#pragma unroll
  for (int j = 0; j < Sh::upt; ++j) {
    int64_t u = base + (int64_t)j * kCastThreads;
    if (u < units) in[j] = load_words<Sh::src_bits>(src + u * (Sh::src_bits / 8));
  }
  if constexpr (ST == F32 && DT == E2M1) {
    // fp32 -> E2M1: a unit's code is only 2 bytes, so a full block regroups
    // its units' codes through LDS and each lane stores 8 contiguous bytes
    // (4 units) -- one 512-byte span per wave instruction instead of 128
    // (2^26 elements, MALL evicted: 51.4 against 54.8 us)
    static_assert(Sh::upt == 4 && Sh::dst_bits == 16, "pack shape");
    __shared__ __attribute__((aligned(16))) uint16_t codes[Sh::upt * kCastThreads];
    const int64_t first = (int64_t)blockIdx.x * Sh::upt * kCastThreads;
    if (first + Sh::upt * kCastThreads <= units) {
#pragma unroll
      for (int j = 0; j < Sh::upt; ++j) {
        uint32_t c = 0;
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          c |= convert<ST, DT, SCALED>(get_elem<32>(in[j], i), s, inv_s) << (4 * i);
        codes[threadIdx.x + j * kCastThreads] = (uint16_t)c;
      }
      __syncthreads();
      const u32x2 v = reinterpret_cast<const u32x2*>(codes)[threadIdx.x];
      __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(dst + first * 2) + threadIdx.x);
    } else {
#pragma unroll
      for (int j = 0; j < Sh::upt; ++j) {
        int64_t u = base + (int64_t)j * kCastThreads;
        if (u < units) {
          uint32_t c = 0;
#pragma unroll
          for (int i = 0; i < EPL; ++i)
            c |= convert<ST, DT, SCALED>(get_elem<32>(in[j], i), s, inv_s) << (4 * i);
          __builtin_nontemporal_store((uint16_t)c, reinterpret_cast<uint16_t*>(dst + u * 2));
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < Sh::upt; ++j) {
      int64_t u = base + (int64_t)j * kCastThreads;
      if (u < units) {
        Words<Sh::dst_words> out;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          uint32_t c = get_elem<dtype_bits(ST)>(in[j], i);
          put_elem<dtype_bits(DT)>(out, i, convert<ST, DT, SCALED>(c, s, inv_s));
        }
        store_words<Sh::dst_bits>(dst + u * (Sh::dst_bits / 8), out);
      }
    }
  }

  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) {
    for (int64_t i = units * EPL; i < n; ++i) {
      uint32_t c = convert<ST, DT, SCALED>(load_scalar<ST>(src, i), s, inv_s);
      if constexpr (dtype_bits(DT) == 32) reinterpret_cast<uint32_t*>(dst)[i] = c;
      else if constexpr (dtype_bits(DT) == 16) reinterpret_cast<uint16_t*>(dst)[i] = (uint16_t)c;
      else if constexpr (dtype_bits(DT) == 8) dst[i] = (uint8_t)c;
      else {
        // units * EPL is even, so pairs start at even i; the odd tail pads +0.
        if ((i & 1) == 0) dst[i >> 1] = (uint8_t)(c & 0xFu);
        else dst[i >> 1] |= (uint8_t)((c & 0xFu) << 4);
      }
    }
  }
}

// ---- amax ----

// One 1024-thread workgroup per CU (16 waves, 4 x 16-byte loads in flight
// per lane): every workgroup ends with one atomicMax on the same word, and
// those serialise at the L2 (about 4.4 ns each), so the grid is kept to one
// workgroup per CU.  Measured on 2^28 fp32 with the MALL evicted: 165 us
// (6.5 TB/s), against 196-199 us with 256-thread workgroups, 8 per CU; a
// reduction without any atomic reads at 6.9 TB/s.
constexpr int kAmaxThreads = 1024;
constexpr int kAmaxUnroll = 4;

template <int ST>
__device__ __forceinline__ uint32_t abs_bits_or_zero(uint32_t c) {
  uint32_t a = decode<ST>(c) & 0x7FFFFFFFu;
  return a > 0x7F800000u ? 0u : a;  // NaN ignored
}

// Grid-stride max of |x| over 16-byte chunks; non-negative fp32 magnitudes
// order like their bit patterns, so the running max and the final atomicMax
// work on uint32.  *out must hold 0 (or a smaller magnitude) on entry.
template <int ST>
__global__ __launch_bounds__(kAmaxThreads) void amax_kernel(const uint8_t* __restrict__ src,
                                                            int64_t n, uint32_t* out) {
  constexpr int EPC = 128 / dtype_bits(ST);  // elements per 16-byte chunk
  const int64_t chunks = n / EPC;
  const u32x4* p = reinterpret_cast<const u32x4*>(src);
  const int64_t stride = (int64_t)gridDim.x * kAmaxThreads;
  uint32_t m = 0;
  int64_t c = (int64_t)blockIdx.x * kAmaxThreads + threadIdx.x;
  for (; c + (kAmaxUnroll - 1) * stride < chunks; c += kAmaxUnroll * stride) {
    u32x4 q[kAmaxUnroll];
#pragma unroll
    for (int j = 0; j < kAmaxUnroll; ++j) q[j] = __builtin_nontemporal_load(p + c + j * stride);
#pragma unroll
    for (int j = 0; j < kAmaxUnroll; ++j) {
      Words<4> v{{q[j].x, q[j].y, q[j].z, q[j].w}};
#pragma unroll
      for (int i = 0; i < EPC; ++i) m = max(m, abs_bits_or_zero<ST>(get_elem<dtype_bits(ST)>(v, i)));
    }
  }
  for (; c < chunks; c += stride) {
    u32x4 q = __builtin_nontemporal_load(p + c);
    Words<4> v{{q.x, q.y, q.z, q.w}};
#pragma unroll
    for (int i = 0; i < EPC; ++i) m = max(m, abs_bits_or_zero<ST>(get_elem<dtype_bits(ST)>(v, i)));
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    for (int64_t i = chunks * EPC; i < n; ++i) m = max(m, abs_bits_or_zero<ST>(load_scalar<ST>(src, i)));
  }
  // wave64 reduction, then across the block's waves through LDS
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
  __shared__ uint32_t wave_max[kAmaxThreads / 64];
  if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t b = wave_max[0];
#pragma unroll
    for (int w = 1; w < kAmaxThreads / 64; ++w) b = max(b, wave_max[w]);
    atomicMax(out, b);
  }
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, int count) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) p[i] = v;
}

int fill_u32_launch(uint32_t* p, uint32_t v, int count, hipStream_t stream) {
  if (count <= 0) return NOVAQ_OK;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream,
                     p, v, count);
  return check_launch();
}

template <int DT>
__global__ void scale_from_amax_kernel(const float* amax, float* scale) {
  if (threadIdx.x == 0) *scale = scale_from_amax_dev<DT>(*amax);
}

// ---- launchers ----

template <int ST, int DT, int SMODE>
static int launch_cast(const void* src, void* dst, int64_t n, const float* scale,
                       float* scale_out, hipStream_t stream) {
  using Sh = CastShape<ST, DT>;
  int64_t units = n / Sh::epl;
  int64_t per_block = (int64_t)Sh::upt * kCastThreads;
  int64_t blocks = (units + per_block - 1) / per_block;
  if (blocks < 1) blocks = 1;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  hipLaunchKernelGGL((cast_kernel<ST, DT, SMODE>), dim3((unsigned)blocks), dim3(kCastThreads),
                     0, stream, static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst),
                     n, scale, scale_out);
  return check_launch();
}

template <int ST, int DT>
static int dispatch_smode(int smode, const void* src, void* dst, int64_t n,
                          const float* scale, float* scale_out, hipStream_t stream) {
  if constexpr (is_quant(ST) || is_quant(DT)) {
    if (smode == 1) return launch_cast<ST, DT, 1>(src, dst, n, scale, nullptr, stream);
    if (smode == 2) {
      // the scale is derived from an amax only when quantizing
      if constexpr (is_quant(DT)) return launch_cast<ST, DT, 2>(src, dst, n, scale, scale_out, stream);
      else return NOVAQ_EINVAL;
    }
  } else {
    if (smode != 0) return NOVAQ_EINVAL;
  }
  return launch_cast<ST, DT, 0>(src, dst, n, nullptr, nullptr, stream);
}

template <int ST>
static int dispatch_dst(int dt, int smode, const void* src, void* dst, int64_t n,
                        const float* scale, float* scale_out, hipStream_t stream) {
  switch (dt) {
    case F32: return dispatch_smode<ST, F32>(smode, src, dst, n, scale, scale_out, stream);
    case F16: return dispatch_smode<ST, F16>(smode, src, dst, n, scale, scale_out, stream);
    case BF16: return dispatch_smode<ST, BF16>(smode, src, dst, n, scale, scale_out, stream);
    case E4M3: return dispatch_smode<ST, E4M3>(smode, src, dst, n, scale, scale_out, stream);
    case E5M2: return dispatch_smode<ST, E5M2>(smode, src, dst, n, scale, scale_out, stream);
    case E2M1: return dispatch_smode<ST, E2M1>(smode, src, dst, n, scale, scale_out, stream);
    default: return NOVAQ_EDTYPE;
  }
}

template <int QT>
static int dispatch_from_quant(int dt, int smode, const void* src, void* dst, int64_t n,
                               const float* scale, hipStream_t stream) {
  switch (dt) {
    case F32: return dispatch_smode<QT, F32>(smode, src, dst, n, scale, nullptr, stream);
    case F16: return dispatch_smode<QT, F16>(smode, src, dst, n, scale, nullptr, stream);
    case BF16: return dispatch_smode<QT, BF16>(smode, src, dst, n, scale, nullptr, stream);
    default: return NOVAQ_EDTYPE;  // quantized -> quantized
  }
}

int cast_launch(const void* src, int st, void* dst, int dt, int64_t n, int smode,
                const float* scale, float* scale_out, hipStream_t stream) {
  switch (st) {
    case F32: return dispatch_dst<F32>(dt, smode, src, dst, n, scale, scale_out, stream);
    case F16: return dispatch_dst<F16>(dt, smode, src, dst, n, scale, scale_out, stream);
    case BF16: return dispatch_dst<BF16>(dt, smode, src, dst, n, scale, scale_out, stream);
    case E4M3: return dispatch_from_quant<E4M3>(dt, smode, src, dst, n, scale, stream);
    case E5M2: return dispatch_from_quant<E5M2>(dt, smode, src, dst, n, scale, stream);
    case E2M1: return dispatch_from_quant<E2M1>(dt, smode, src, dst, n, scale, stream);
    default: return NOVAQ_EDTYPE;
  }
}

template <int ST>
static int launch_amax(const void* x, int64_t n, float* amax, hipStream_t stream) {
  hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, stream,
                     reinterpret_cast<uint32_t*>(amax), 0u, 1);
  int rc = check_launch();
  if (rc != NOVAQ_OK) return rc;
  constexpr int EPC = 128 / dtype_bits(ST);
  int64_t chunks = n / EPC;
  int64_t want = (chunks + (int64_t)kAmaxThreads * kAmaxUnroll - 1) / ((int64_t)kAmaxThreads * kAmaxUnroll);
  int64_t cap = (int64_t)device_cu_count();
  int64_t blocks = want < 1 ? 1 : (want > cap ? cap : want);
  hipLaunchKernelGGL((amax_kernel<ST>), dim3((unsigned)blocks), dim3(kAmaxThreads), 0, stream,
                     static_cast<const uint8_t*>(x), n, reinterpret_cast<uint32_t*>(amax));
  return check_launch();
}

int amax_launch(const void* x, int dt, int64_t n, float* amax, hipStream_t stream) {
  switch (dt) {
    case F32: return launch_amax<F32>(x, n, amax, stream);
    case F16: return launch_amax<F16>(x, n, amax, stream);
    case BF16: return launch_amax<BF16>(x, n, amax, stream);
    default: return NOVAQ_EDTYPE;
  }
}

int scale_from_amax_launch(const float* amax, int dt, float* scale, hipStream_t stream) {
  switch (dt) {
    case E4M3: hipLaunchKernelGGL(scale_from_amax_kernel<E4M3>, dim3(1), dim3(64), 0, stream, amax, scale); break;
    case E5M2: hipLaunchKernelGGL(scale_from_amax_kernel<E5M2>, dim3(1), dim3(64), 0, stream, amax, scale); break;
    case E2M1: hipLaunchKernelGGL(scale_from_amax_kernel<E2M1>, dim3(1), dim3(64), 0, stream, amax, scale); break;
    default: return NOVAQ_EDTYPE;
  }
  return check_launch();
}

}  // namespace novaq
