// Decoding on CDNA4 (gfx950): attention of one new token per row over a fixed-capacity KV ring.
//
// Semantics (reference vesper/attention.py:62-139, :298-338): a token at position p lives in slot
// p % W; slots are not in age order. The query at position p attends the ring slots that are valid
// and hold a position in (p - W, p], plus the new token itself, which is attended exactly once
// from its own argument; only then is the new token written into its slot (keys, values, position,
// valid flag). Query head h reads KV head h / (H / HKV); scale 1/sqrt(D) (passed in).
//
// ring_attn_kernel: one workgroup per (b, KV head) serves the G = H / HKV query heads of that
// group, so each ring row is read from HBM once per step. D/8 lanes share a key row (16-byte
// pieces; D is the head width rounded up to a power of two, and with PAD the lanes past the real
// width dk load nothing and hold zeros); a thread takes KPT keys of a batch and issues all of their K and V loads before any
// arithmetic, so the whole window of the head is in flight at once (W = 512 at D = 64 is one
// batch). Each thread keeps, per query head, an online softmax over its own keys (running max,
// sum and weighted values, base-2 exponent); the partial states merge across the key groups of a
// wave with lane shuffles and across the waves through LDS, in a fixed order.
//
// The write: a workgroup writes its own KV head's key and value into slot p % W after all of its
// reads (no other workgroup reads that head). The slot's position and valid flag are shared by the
// HKV workgroups of row b, so the last of them to finish reading the row's positions and flags (a
// per-row arrival counter in the caller's workspace) writes them and resets the counter to zero:
// every workgroup of the row has read the old position and flag by then, whatever order the
// workgroups ran in.
#include <mutex>
#include <type_traits>

#include "common.h"
#include "vesper_kernels.h"

namespace vsp {
namespace {

constexpr int kMaxGroup = 8;

// The workgroup shape by GM, the query heads per KV head rounded up to a power of two (register
// arrays are sized by it): groups of up to two query heads run 1024 threads with four keys each
// (many waves per CU with few loads each stream the window faster than fewer waves with many loads:
// 24.6 against 25.1 us per decode step with the ring read from HBM); wider groups run 256 threads
// with eight keys each, so the per-head softmax states still fit in registers.
template <typename T> struct Ring8 {
  typedef T V8 __attribute__((ext_vector_type(8)));
};

template <int GM> struct RingShape {
  static constexpr int NT = GM <= 2 ? 1024 : 256;  // threads
  static constexpr int KPT = GM <= 2 ? 4 : 8;      // keys per thread per batch
};

// Eight ring elements as the queries' type: the ring's own type is either the queries' (one 16-byte
// load) or float32 (two, each element rounded to nearest even, as the reference's autocast casts an
// fp32 ring to the query dtype, attention.py:325). The loads are nontemporal: a decode step reads
// each ring once, and a column's rings (one a pass) together outgrow the MALL, so they stream.
template <typename T, typename R>
__device__ __forceinline__ typename Ring8<T>::V8 load_ring8(const R* p) {
  typedef typename Ring8<T>::V8 V8;
  if constexpr (sizeof(R) == sizeof(T)) {
    return __builtin_nontemporal_load(reinterpret_cast<const V8*>(p));
  } else {
    const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + 1);
    V8 x;
    x[0] = from_f32<T>(a[0]); x[1] = from_f32<T>(a[1]); x[2] = from_f32<T>(a[2]); x[3] = from_f32<T>(a[3]);
    x[4] = from_f32<T>(b[0]); x[5] = from_f32<T>(b[1]); x[6] = from_f32<T>(b[2]); x[7] = from_f32<T>(b[3]);
    return x;
  }
}
// The new token's eight elements into the ring (widened exactly when the ring is float32).
template <typename T, typename R>
__device__ __forceinline__ void store_ring8(R* p, const typename Ring8<T>::V8& x) {
  if constexpr (sizeof(R) == sizeof(T)) {
    *reinterpret_cast<typename Ring8<T>::V8*>(p) = x;
  } else {
    reinterpret_cast<float4*>(p)[0] = make_float4(to_f32(x[0]), to_f32(x[1]), to_f32(x[2]), to_f32(x[3]));
    reinterpret_cast<float4*>(p)[1] = make_float4(to_f32(x[4]), to_f32(x[5]), to_f32(x[6]), to_f32(x[7]));
  }
}

template <typename T, typename R, int D, int GM, bool PAD>
__global__ __launch_bounds__(RingShape<GM>::NT) void ring_attn_kernel(
    const T* __restrict__ q, const T* __restrict__ knew, const T* __restrict__ vnew, const int64_t* __restrict__ pos,
    R* ring_k, R* ring_v, int64_t* ring_pos, uint8_t* ring_valid, T* __restrict__ o, const uint8_t* __restrict__ active,
    uint32_t* __restrict__ counters, int H, int HKV, int W, float scale_log2, int write, int dk_arg) {
  constexpr int NT = RingShape<GM>::NT;
  constexpr int NW = NT / 64;              // waves
  constexpr int KL = D / 8;                // lanes per key row
  constexpr int KPP = NT / KL;             // keys per pass of the workgroup
  constexpr int KPT = RingShape<GM>::KPT;  // keys per thread per batch
  constexpr int BATCH = KPP * KPT;
  constexpr int VPT = (BATCH + NT - 1) / NT;  // visibility flags computed per thread per batch
  constexpr bool kQReg = GM <= 2;          // query pieces in registers (else read from LDS per key)
  typedef T V8 __attribute__((ext_vector_type(8)));
  using P2 = typename Dot2<T>::P2;
  __shared__ __align__(16) T sq[GM][D];
  __shared__ uint8_t svis[BATCH];
  __shared__ float smerge[NW][GM][2 + D];

  const int b = blockIdx.x / HKV, kvh = blockIdx.x - b * HKV;
  const int G = H / HKV;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int part = tid % KL, kg = tid / KL;
  const int dk = PAD ? dk_arg : D;       // the real head width (a multiple of 8, at most D)
  const bool live = !PAD || 8 * part < dk;  // this lane's 8 features exist
  const int64_t p = pos[b];
  const size_t row_stride = (size_t)HKV * dk;
  const size_t head_off = ((size_t)b * W * HKV + kvh) * dk + 8 * part;
  T* out = o + ((size_t)b * H + (size_t)kvh * G) * dk;
  // An inactive row is computed like an active one and stores zeros, so no wait on its flag delays
  // the row's loads; its token is still written.
  {
    float m[GM], l[GM], acc[GM][8];
#pragma unroll
    for (int gi = 0; gi < GM; ++gi) {
      m[gi] = -1e30f;  // finite: a thread that sees no key keeps l = 0 and merges as nothing
      l[gi] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[gi][e] = 0.f;
    }
    V8 qr[kQReg ? GM : 1];
    // one batch of n <= KPT keys of this thread (scores sc, values vr) folded into the running state
    auto fold = [&](float (&sc)[GM][KPT], const V8* vr, int n) {
#pragma unroll
      for (int gi = 0; gi < GM; ++gi) {
        float mb = sc[gi][0];
#pragma unroll
        for (int i = 1; i < KPT; ++i)
          if (i < n) mb = fmaxf(mb, sc[gi][i]);
        const float mn = fmaxf(m[gi], mb);
        const float a = __builtin_amdgcn_exp2f(m[gi] - mn);
        l[gi] *= a;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[gi][e] *= a;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
          if (i < n) {
            const float pj = __builtin_amdgcn_exp2f(sc[gi][i] - mn);
            l[gi] += pj;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[gi][e] += pj * to_f32(vr[i][e]);
          }
        }
        m[gi] = mn;
      }
    };
    auto dot = [&](int gi, const V8& kv) {
      V8 qv;
      if constexpr (kQReg) {
        qv = qr[kQReg ? gi : 0];
      } else {
        qv = *reinterpret_cast<const V8*>(&sq[gi][8 * part]);
      }
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e += 2) s = Dot2<T>::run(P2{kv[e], kv[e + 1]}, P2{qv[e], qv[e + 1]}, s);
      return group_sum<KL>(s) * scale_log2;
    };

    const R* kb = ring_k + head_off;
    const R* vb = ring_v + head_off;
    for (int j0 = 0; j0 < W; j0 += BATCH) {
      // positions and flags first, then every key and value load of the batch: waiting for the
      // first does not wait for the rest (the load counter retires in order)
      int64_t rp[VPT];
      uint8_t rv[VPT];
#pragma unroll
      for (int u = 0; u < VPT; ++u) {
        const int j = min(j0 + tid + NT * u, W - 1);
        rp[u] = ring_pos[(size_t)b * W + j];
        rv[u] = ring_valid[(size_t)b * W + j];
      }
      V8 kr[KPT], vr[KPT];
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const int j = min(j0 + kg + i * KPP, W - 1);  // keys past W re-read row W - 1, masked below
        if (live) {
          kr[i] = load_ring8<T>(kb + (size_t)j * row_stride);
          vr[i] = load_ring8<T>(vb + (size_t)j * row_stride);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) kr[i][e] = vr[i][e] = from_f32<T>(0.f);
        }
      }
      if (j0 == 0) {  // the group's query heads (heads past G are zero: their results are never stored)
        const T* qb = q + ((size_t)b * H + (size_t)kvh * G) * dk;
        if constexpr (kQReg) {
#pragma unroll
          for (int gi = 0; gi < GM; ++gi) {
            if (gi < G && live) {
              qr[gi] = *reinterpret_cast<const V8*>(qb + gi * dk + 8 * part);
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) qr[gi][e] = from_f32<T>(0.f);
            }
          }
        } else {
          for (int i = tid; i < GM * D; i += NT) {
            const int gi = i / D, d = i % D;
            sq[gi][d] = gi < G && d < dk ? qb[gi * dk + d] : from_f32<T>(0.f);
          }
        }
      }
      __syncthreads();  // the previous batch's flags are read (and sq is written)
#pragma unroll
      for (int u = 0; u < VPT; ++u) {
        const int jj = tid + NT * u;
        if (jj < BATCH) svis[jj] = (j0 + jj < W && rv[u] != 0 && rp[u] <= p && rp[u] > p - W) ? 1 : 0;
      }
      __syncthreads();
      if (write && p >= 0 && tid == 0 && j0 + BATCH >= W) {
        // This workgroup has read every position and flag of the row it will read (the last batch's
        // are in LDS now), so it reports in; the row's last workgroup to report writes the slot's
        // position and flag. No fence is needed on either side: the loads reporting here have
        // returned (their values were consumed before the barrier), so a store issued after this
        // increment is observed cannot reach them, and what is written here is read by later
        // launches only. The counter is a relaxed device-scope atomic, coherent across the XCDs'
        // L2s (an agent-scope fence would write back the whole L2, dearer than the attention).
        // Reporting here rather than at the end hides the atomic's round trip behind the K/V loads.
        const uint32_t arrived = __hip_atomic_fetch_add(&counters[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (arrived == (uint32_t)(HKV - 1)) {
          const int slot = (int)(p % W);
          ring_pos[(size_t)b * W + slot] = p;
          ring_valid[(size_t)b * W + slot] = 1;
          __hip_atomic_store(&counters[b], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      float sc[GM][KPT];
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const bool vis = svis[kg + i * KPP] != 0;
#pragma unroll
        for (int gi = 0; gi < GM; ++gi) {
          const float sv = dot(gi, kr[i]);
          sc[gi][i] = vis ? sv : -INFINITY;
        }
      }
      fold(sc, vr, KPT);
    }
    if (kg == 0) {  // the new token, always visible
      V8 kn, vn[KPT];
      if (live) {
        kn = *reinterpret_cast<const V8*>(knew + ((size_t)b * HKV + kvh) * dk + 8 * part);
        vn[0] = *reinterpret_cast<const V8*>(vnew + ((size_t)b * HKV + kvh) * dk + 8 * part);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) kn[e] = vn[0][e] = from_f32<T>(0.f);
      }
      float sc[GM][KPT];
#pragma unroll
      for (int gi = 0; gi < GM; ++gi) sc[gi][0] = dot(gi, kn);
      fold(sc, vn, 1);
    }

    // merge the partial softmax states: key groups of a wave, then the waves
#pragma unroll
    for (int gi = 0; gi < GM; ++gi) {
#pragma unroll
      for (int off = KL; off < 64; off <<= 1) {
        const float mo = __shfl_xor(m[gi], off);
        const float lo = __shfl_xor(l[gi], off);
        const float mn = fmaxf(m[gi], mo);
        const float a = __builtin_amdgcn_exp2f(m[gi] - mn), c = __builtin_amdgcn_exp2f(mo - mn);
        l[gi] = l[gi] * a + lo * c;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[gi][e] = acc[gi][e] * a + __shfl_xor(acc[gi][e], off) * c;
        m[gi] = mn;
      }
      if (lane < KL) {
        if (part == 0) {
          smerge[wv][gi][0] = m[gi];
          smerge[wv][gi][1] = l[gi];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) smerge[wv][gi][2 + 8 * part + e] = acc[gi][e];
      }
    }
    __syncthreads();
    const bool on = active == nullptr || active[b] != 0;
    for (int i = tid; i < G * dk; i += NT) {
      const int gi = i / dk, d = i - gi * dk;
      float mx = smerge[0][gi][0];
#pragma unroll
      for (int w = 1; w < NW; ++w) mx = fmaxf(mx, smerge[w][gi][0]);
      float lsum = 0.f, num = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float a = __builtin_amdgcn_exp2f(smerge[w][gi][0] - mx);
        lsum += smerge[w][gi][1] * a;
        num += smerge[w][gi][2 + d] * a;
      }
      out[i] = from_f32<T>(on ? num / lsum : 0.f);
    }
  }

  if (!write || p < 0) return;  // a negative position is refused by the host wrapper
  __syncthreads();              // every read of this workgroup is done
  const int slot = (int)(p % W);
  const size_t dst = ((size_t)b * W + slot) * row_stride + (size_t)kvh * dk;
  const size_t src = ((size_t)b * HKV + kvh) * dk;
  if (tid < KL) {
    if (8 * tid < dk) store_ring8<T>(ring_k + dst + 8 * tid, *reinterpret_cast<const V8*>(knew + src + 8 * tid));
  } else if (tid < 2 * KL) {
    const int pp = tid - KL;
    if (8 * pp < dk) store_ring8<T>(ring_v + dst + 8 * pp, *reinterpret_cast<const V8*>(vnew + src + 8 * pp));
  }
}

// Head widths the ring kernel takes: multiples of 8 (16-byte rows) up to 256; the powers of two run
// their own shape, the others the next power of two's lanes with the lanes past the width idle.
bool ring_width(int D) { return D >= 8 && D <= 256 && D % 8 == 0; }

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

template <typename T, typename R = T>
int ring_attn(const T* q, const T* knew, const T* vnew, const int64_t* pos, R* ring_k, R* ring_v, int64_t* ring_pos,
              uint8_t* ring_valid, T* o, const uint8_t* active, void* workspace, size_t ws_bytes, int B, int H, int HKV,
              int D, int W, float scale, int write, void* stream_ptr, const char* who) {
  if (B < 0 || H < 1 || HKV < 1 || W < 1) return fail(ERR_ARG, "%s: bad sizes B=%d H=%d HKV=%d W=%d", who, B, H, HKV, W);
  if (H % HKV != 0) return fail(ERR_ARG, "%s: %d query heads are not a multiple of %d KV heads", who, H, HKV);
  if (H / HKV > kMaxGroup) return fail(ERR_UNSUPPORTED, "%s: %d query heads per KV head (at most %d)", who, H / HKV, kMaxGroup);
  if (!ring_width(D)) return fail(ERR_UNSUPPORTED, "%s: head dimension %d (kernels: multiples of 8 up to 256)", who, D);
  if (B == 0) return OK;
  if (!q || !knew || !vnew || !pos || !ring_k || !ring_v || !ring_pos || !ring_valid || !o)
    return fail(ERR_ARG, "%s: null pointer", who);
  if (!aligned16(q) || !aligned16(knew) || !aligned16(vnew) || !aligned16(ring_k) || !aligned16(ring_v))
    return fail(ERR_ARG, "%s: q, k, v and the ring's keys and values must be 16-byte aligned", who);
  if (write && (workspace == nullptr || ws_bytes < (size_t)B * sizeof(uint32_t)))
    return fail(ERR_ARG, "%s: workspace of %zu bytes given, %zu needed", who, workspace ? ws_bytes : (size_t)0,
                (size_t)B * sizeof(uint32_t));
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  const float scale_log2 = scale * 1.4426950408889634f;
  uint32_t* counters = static_cast<uint32_t*>(workspace);
  dim3 grid((unsigned)(B * HKV));
  const int G = H / HKV;
  auto go = [&](auto kern, int nt) {
    hipLaunchKernelGGL(kern, grid, dim3(nt), 0, stream, q, knew, vnew, pos, ring_k, ring_v, ring_pos, ring_valid, o,
                       active, counters, H, HKV, W, scale_log2, write, D);
  };
  auto by_group = [&](auto dtag, auto padtag) {
    constexpr int Dc = decltype(dtag)::value;
    constexpr bool Pc = decltype(padtag)::value;
    if (G == 1) go(ring_attn_kernel<T, R, Dc, 1, Pc>, RingShape<1>::NT);
    else if (G == 2) go(ring_attn_kernel<T, R, Dc, 2, Pc>, RingShape<2>::NT);
    else if (G <= 4) go(ring_attn_kernel<T, R, Dc, 4, Pc>, RingShape<4>::NT);
    else go(ring_attn_kernel<T, R, Dc, 8, Pc>, RingShape<8>::NT);
  };
  auto by_width = [&](auto padtag) {
    const int Dp = D <= 8 ? 8 : D <= 16 ? 16 : D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256;
    switch (Dp) {
      case 8: by_group(std::integral_constant<int, 8>{}, padtag); break;
      case 16: by_group(std::integral_constant<int, 16>{}, padtag); break;
      case 32: by_group(std::integral_constant<int, 32>{}, padtag); break;
      case 64: by_group(std::integral_constant<int, 64>{}, padtag); break;
      case 128: by_group(std::integral_constant<int, 128>{}, padtag); break;
      default: by_group(std::integral_constant<int, 256>{}, padtag); break;
    }
  };
  if ((D & (D - 1)) == 0) by_width(std::false_type{});
  else by_width(std::true_type{});
  return check_launch(who);
}

}  // namespace

// ---- the allocation-free entry's static scratch -------------------------------------------------
// The per-row arrival counters of the in-kernel ring write, for callers that cannot allocate (code
// under graph capture, serving loops): a file-scope device array, one copy per GPU, alive until the
// process ends. Host code never passes the array's name to a kernel (in host code it is a host-side
// stand-in, not a device address): ring_scratch_init takes the current device's address with
// hipGetSymbolAddress and the entry point uses that address. Only the current device is touched:
// vsp_init sets up the device current when it runs, and the entry point sets up any other device
// on its first call there (a process that uses one GPU never creates a context on another).
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint32_t scratch[kNoAllocMaxRows];
uint32_t* g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mutex;

// zeroes the counters on a stream (a kernel, not a memset: the first call on a device may be
// captured into a graph)
__global__ __launch_bounds__(256) void zero_counters_kernel(uint32_t* c, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) c[i] = 0u;
}

// The current device's scratch address, set up on first use; null (with the error set) on failure.
// `stream` null: zeroed synchronously (vsp_init); otherwise zeroed by a kernel on that stream,
// ahead of the caller's launch.
uint32_t* scratch_of_current(hipStream_t stream, bool sync_zero) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) {
    fail(ERR_LAUNCH, "static scratch: hipGetDevice: %s", hipGetErrorString(err));
    return nullptr;
  }
  if (device < 0 || device >= kMaxDevices) {
    fail(ERR_UNSUPPORTED, "static scratch: device %d beyond the %d this build tracks", device, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[device] != nullptr) return g_scratch[device];
  void* ptr = nullptr;
  err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (err != hipSuccess) {
    fail(ERR_LAUNCH, "static scratch on device %d: hipGetSymbolAddress: %s", device, hipGetErrorString(err));
    return nullptr;
  }
  // the counters start at zero; every call that writes the ring leaves them zero again
  if (sync_zero) {
    err = hipMemset(ptr, 0, sizeof(scratch));
  } else {
    hipLaunchKernelGGL(zero_counters_kernel, dim3((kNoAllocMaxRows + 255) / 256), dim3(256), 0, stream,
                       static_cast<uint32_t*>(ptr), kNoAllocMaxRows);
    err = hipGetLastError();
  }
  if (err != hipSuccess) {
    fail(ERR_LAUNCH, "static scratch on device %d: zeroing: %s", device, hipGetErrorString(err));
    return nullptr;
  }
  g_scratch[device] = static_cast<uint32_t*>(ptr);
  return g_scratch[device];
}

int ring_scratch_init() { return scratch_of_current(nullptr, true) != nullptr ? OK : ERR_LAUNCH; }

}  // namespace vsp

extern "C" size_t vsp_ring_attn_workspace_bytes(int B) { return B > 0 ? (size_t)B * sizeof(uint32_t) : 0; }

extern "C" int vsp_ring_attn_noalloc_bf16(const void* q, const void* k, const void* v, const int64_t* pos,
                                          void* ring_k, void* ring_v, int64_t* ring_pos, uint8_t* ring_valid, void* o,
                                          const uint8_t* active, int B, int H, int HKV, int D, int window, float scale,
                                          int write, void* stream) {
  const char* who = "vsp_ring_attn_noalloc_bf16";
  if (B > vsp::kNoAllocMaxRows)
    return vsp::fail(vsp::ERR_ARG, "%s: %d rows exceed the static scratch's %d", who, B, vsp::kNoAllocMaxRows);
  uint32_t* counters = vsp::scratch_of_current(reinterpret_cast<hipStream_t>(stream), false);
  if (counters == nullptr) return vsp::ERR_LAUNCH;
  return vsp::ring_attn<__bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                                static_cast<const __bf16*>(v), pos, static_cast<__bf16*>(ring_k),
                                static_cast<__bf16*>(ring_v), ring_pos, ring_valid, static_cast<__bf16*>(o), active,
                                counters, sizeof(uint32_t) * (size_t)vsp::kNoAllocMaxRows, B, H, HKV, D,
                                window, scale, write, stream, who);
}

extern "C" int vsp_ring_attn_bf16(const void* q, const void* k, const void* v, const int64_t* pos, void* ring_k,
                                  void* ring_v, int64_t* ring_pos, uint8_t* ring_valid, void* o,
                                  const uint8_t* active, void* workspace, size_t workspace_bytes, int B, int H, int HKV,
                                  int D, int window, float scale, int write, void* stream) {
  return vsp::ring_attn<__bf16>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                                static_cast<const __bf16*>(v), pos, static_cast<__bf16*>(ring_k),
                                static_cast<__bf16*>(ring_v), ring_pos, ring_valid, static_cast<__bf16*>(o), active,
                                workspace, workspace_bytes, B, H, HKV, D, window, scale, write, stream,
                                "vsp_ring_attn_bf16");
}

extern "C" int vsp_ring_attn_f16(const void* q, const void* k, const void* v, const int64_t* pos, void* ring_k,
                                 void* ring_v, int64_t* ring_pos, uint8_t* ring_valid, void* o, const uint8_t* active,
                                 void* workspace, size_t workspace_bytes, int B, int H, int HKV, int D, int window,
                                 float scale, int write, void* stream) {
  return vsp::ring_attn<_Float16>(static_cast<const _Float16*>(q), static_cast<const _Float16*>(k),
                                  static_cast<const _Float16*>(v), pos, static_cast<_Float16*>(ring_k),
                                  static_cast<_Float16*>(ring_v), ring_pos, ring_valid, static_cast<_Float16*>(o),
                                  active, workspace, workspace_bytes, B, H, HKV, D, window, scale, write, stream,
                                  "vsp_ring_attn_f16");
}

// The ring in float32 with bf16 / fp16 queries: the ring the reference's captured decoder allocates
// (init_states(1, torch.float32, ...), vesper/decode.py:81,85; column.py:492), whose keys and values
// attend_ring casts to the queries' dtype (attention.py:325). Each ring element is rounded to the
// queries' dtype as it is loaded; the new token is written into its slot widened to float32.
extern "C" int vsp_ring_attn_bf16_ring_f32(const void* q, const void* k, const void* v, const int64_t* pos,
                                           float* ring_k, float* ring_v, int64_t* ring_pos, uint8_t* ring_valid,
                                           void* o, const uint8_t* active, void* workspace, size_t workspace_bytes,
                                           int B, int H, int HKV, int D, int window, float scale, int write,
                                           void* stream) {
  return vsp::ring_attn<__bf16, float>(static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                                       static_cast<const __bf16*>(v), pos, ring_k, ring_v, ring_pos, ring_valid,
                                       static_cast<__bf16*>(o), active, workspace, workspace_bytes, B, H, HKV, D,
                                       window, scale, write, stream, "vsp_ring_attn_bf16_ring_f32");
}

extern "C" int vsp_ring_attn_f16_ring_f32(const void* q, const void* k, const void* v, const int64_t* pos,
                                          float* ring_k, float* ring_v, int64_t* ring_pos, uint8_t* ring_valid,
                                          void* o, const uint8_t* active, void* workspace, size_t workspace_bytes,
                                          int B, int H, int HKV, int D, int window, float scale, int write,
                                          void* stream) {
  return vsp::ring_attn<_Float16, float>(static_cast<const _Float16*>(q), static_cast<const _Float16*>(k),
                                         static_cast<const _Float16*>(v), pos, ring_k, ring_v, ring_pos, ring_valid,
                                         static_cast<_Float16*>(o), active, workspace, workspace_bytes, B, H, HKV, D,
                                         window, scale, write, stream, "vsp_ring_attn_f16_ring_f32");
}
