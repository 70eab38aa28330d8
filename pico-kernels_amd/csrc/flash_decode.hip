// Split-KV single-query attention for decode (the FlashDecoding scheme of the reference's
// flash_decoding.py:47-115): for every (batch b, head h) the cached keys/values are cut into
// splits of `split` rows; each split produces (m, l, acc) = (max score, sum of
// exp(score - m), sum of exp(score - m) * v) in fp32, and the splits are combined as
// m* = max m_s, l* = sum l_s e^(m_s - m*), o = sum acc_s e^(m_s - m*) / l*, in split order.
//
// Split kernel: one workgroup of NT threads per (b*H + h, split). Lane (c, r), c = t % CL with
// CL = D / 8, reads 16 bytes (8 head dims) of key/value rows i * RG + r of the split (RG = NT /
// CL row groups), so each wave instruction covers whole contiguous rows. Scores are v_dot2
// partial sums reduced over the CL lanes of a row by shuffles.
//   * Up to 16 passes of RG rows: every lane holds its KPL rows in registers; the split's max
//     is reduced first (shuffles, then LDS across waves) and each exp is taken once against it.
//   * Longer splits: chunks of 8 passes with a running (m, l, acc) per lane (online softmax),
//     rescaled to the split's max once at the end.
// Rows past the split's end (a split that is not a whole number of passes) score -inf and
// read row 0 of the split instead. Sums over lanes and waves follow a fixed order, so results
// are reproducible bit for bit.
//
// Combine: either a second kernel (one workgroup per (b, h)) or, in one launch, the last of
// a (b, h)'s splits to finish: the 1-D grid puts every split of a (b, h) on one XCD (block
// index mod 8 picks the XCD, as for the split-K GEMV), each split stores its partial, waits
// for the stores to reach L2 and bumps the (b, h)'s arrival counter; the workgroup that sees
// S - 1 combines the S partials in split order (the same arithmetic as the combine kernel) and
// resets the counter. Each (b, h)'s partials start on a 128-byte line of their own, so no
// other (b, h)'s combine can have cached part of them.
//
// K and V are fp16 with unit stride along D; the other strides are free (a KV-cache prefix
// view is read in place).
#include "pk_internal.h"

namespace pk {

struct FdParams {
  const pk_half* q;
  int64_t sqb, sqh;
  const pk_half* k;
  int64_t skb, skh, skn;
  const pk_half* v;
  int64_t svb, svh, svn;
  float* partials;     // (B*H) regions of bh_stride floats: S records [m, l, acc[D]]
  unsigned* counters;  // per (b, h) at a 32-uint stride (one-launch form only)
  float* out;          // (B*H, D) fp32
  int B, H, N, split, S, nch;
  int64_t bh_stride;
  float sm_scale;
};

constexpr int kFdChunkPasses = 8;  // passes of RG rows per chunk on the long-split path
constexpr int kFdMaxPasses = 16;   // register-resident passes on the short-split path

// A vector element goes through a scalar before it is reinterpreted: bit-casting the element
// expression directly has been compiled to read element 0 for every j.
__device__ __forceinline__ pk_half2 half2_of(uint32_t w) { return __builtin_bit_cast(pk_half2, w); }

__device__ __forceinline__ float dot8(const pk_u4v a, const pk_u4v b) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t aj = a[j], bj = b[j];
    s = __builtin_amdgcn_fdot2(half2_of(aj), half2_of(bj), s, false);
  }
  return s;
}

// Head dim d of the combined output of one (b, h) whose S partial records start at `part`.
// Loads go out kFdBatch records at a time; the sums still run in split order.
constexpr int kFdBatch = 16;
__device__ __forceinline__ float fd_combine_dim(const float* part, int S, int rec, int d) {
  float mg = -INFINITY;
  for (int s0 = 0; s0 < S; s0 += kFdBatch) {
    float pm[kFdBatch];
#pragma unroll
    for (int i = 0; i < kFdBatch; ++i) pm[i] = s0 + i < S ? part[(s0 + i) * rec] : -INFINITY;
#pragma unroll
    for (int i = 0; i < kFdBatch; ++i) mg = fmaxf(mg, pm[i]);
  }
  float lg = 0.0f, o = 0.0f;
  for (int s0 = 0; s0 < S; s0 += kFdBatch) {
    float pm[kFdBatch], pl[kFdBatch], pa[kFdBatch];
#pragma unroll
    for (int i = 0; i < kFdBatch; ++i) {
      const float* ps = part + (s0 + i < S ? s0 + i : 0) * rec;
      pm[i] = ps[0];
      pl[i] = ps[1];
      pa[i] = ps[2 + d];
    }
#pragma unroll
    for (int i = 0; i < kFdBatch; ++i) {
      if (s0 + i < S) {
        const float alpha = __expf(pm[i] - mg);
        lg = __builtin_fmaf(pl[i], alpha, lg);
        o = __builtin_fmaf(pa[i], alpha, o);
      }
    }
  }
  return o / lg;
}

template <int D, int KPL, int NT, bool CHUNKED, bool FUSED>
__global__ __launch_bounds__(NT) void fd_split_kernel(FdParams p) {
  constexpr int CL = D / 8, RG = NT / CL, NW = NT / 64, ROWS = KPL * RG, REC = 2 + D;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int c = t % CL, r = t / CL;
  int bh, s;
  if constexpr (FUSED) {
    xcd_tile_slice(p.S, bh, s);
    if (bh >= p.B * p.H) return;  // padding of the last group of 8 (b, h)
  } else {
    bh = blockIdx.x;
    s = blockIdx.y;
  }
  const int b = bh / p.H, h = bh % p.H;
  const int64_t n0 = (int64_t)s * p.split;

  const pk_u4v qv = *reinterpret_cast<const pk_u4v*>(p.q + b * p.sqb + h * p.sqh + 8 * c);
  const pk_half* kb = p.k + b * p.skb + h * p.skh + n0 * p.skn + 8 * c;
  const pk_half* vb = p.v + b * p.svb + h * p.svh + n0 * p.svn + 8 * c;

  __shared__ float s_m[NW], s_l[NW], s_acc[NW][D];
  float m = -INFINITY, l = 0.0f;
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  const int nch = CHUNKED ? p.nch : 1;
  for (int ch = 0; ch < nch; ++ch) {
    pk_u4v kr[KPL], vr[KPL];
    bool ok[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int rr = ch * ROWS + i * RG + r;
      ok[i] = rr < p.split;
      const int64_t n = ok[i] ? rr : 0;
      // K and V are read exactly once: non-temporal loads (measured 13% faster on MI355X)
      kr[i] = __builtin_nontemporal_load(reinterpret_cast<const pk_u4v*>(kb + n * p.skn));
      vr[i] = __builtin_nontemporal_load(reinterpret_cast<const pk_u4v*>(vb + n * p.svn));
    }
    // scores of this lane's rows, summed over the CL lanes of each row
    float sc[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      float x = dot8(qv, kr[i]);
#pragma unroll
      for (int o = 1; o < CL; o <<= 1) x += __shfl_xor(x, o, 64);
      sc[i] = ok[i] ? x * p.sm_scale : -INFINITY;
    }
    float mc = sc[0];
#pragma unroll
    for (int i = 1; i < KPL; ++i) mc = fmaxf(mc, sc[i]);
    if constexpr (!CHUNKED) {
      // the split's max: row groups of the wave, then waves (max is order-free)
#pragma unroll
      for (int o = CL; o < 64; o <<= 1) mc = fmaxf(mc, __shfl_xor(mc, o, 64));
      if (lane == 0) s_m[wave] = mc;
      __syncthreads();
      m = s_m[0];
#pragma unroll
      for (int w = 1; w < NW; ++w) m = fmaxf(m, s_m[w]);
    } else {
      // chunk 0 holds a valid row for every lane (the split spans more than one chunk), so
      // m is finite from then on and the first rescale multiplies zeros by exp(-inf) = 0
      const float mn = fmaxf(m, mc);
      const float f = __expf(m - mn);
      l *= f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] *= f;
      m = mn;
    }
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const float pe = __expf(sc[i] - m);
      l += pe;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t vj = vr[i][j];
        const pk_half2 v2 = half2_of(vj);
        acc[2 * j] = __builtin_fmaf(pe, (float)v2[0], acc[2 * j]);
        acc[2 * j + 1] = __builtin_fmaf(pe, (float)v2[1], acc[2 * j + 1]);
      }
    }
  }
  if constexpr (CHUNKED) {
    // rescale every lane's running sums to the split's max
    float mw = m;
#pragma unroll
    for (int o = CL; o < 64; o <<= 1) mw = fmaxf(mw, __shfl_xor(mw, o, 64));
    if (lane == 0) s_m[wave] = mw;
    __syncthreads();
    float ms = s_m[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) ms = fmaxf(ms, s_m[w]);
    const float f = __expf(m - ms);
    l *= f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] *= f;
    m = ms;
  }
  // sum over the row groups of the wave (fixed butterfly), then over waves in order
#pragma unroll
  for (int o = CL; o < 64; o <<= 1) {
    l += __shfl_xor(l, o, 64);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += __shfl_xor(acc[j], o, 64);
  }
  if (lane < CL) {
    if (lane == 0) s_l[wave] = l;
#pragma unroll
    for (int j = 0; j < 8; ++j) s_acc[wave][8 * c + j] = acc[j];
  }
  __syncthreads();
  float* part = p.partials + (int64_t)bh * p.bh_stride;
  float* rec = part + (int64_t)s * REC;
  for (int d = t; d < D; d += NT) {
    float a = s_acc[0][d];
#pragma unroll
    for (int w = 1; w < NW; ++w) a += s_acc[w][d];
    rec[2 + d] = a;
  }
  if (t == 0) {
    float ls = s_l[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) ls += s_l[w];
    rec[0] = m;
    rec[1] = ls;
  }
  if constexpr (FUSED) {
    if (splitk_arrive(p.counters + (int64_t)bh * 32, p.S)) {
      for (int d = t; d < D; d += NT) p.out[(int64_t)bh * D + d] = fd_combine_dim(part, p.S, REC, d);
    }
  }
}

// Combine the S splits of one (b, h) in a launch of its own: thread d owns head dim d.
template <int D>
__global__ __launch_bounds__(D < 64 ? 64 : D) void fd_combine_kernel(FdParams p) {
  const int bh = blockIdx.x, d = threadIdx.x;
  if (d < D) p.out[(int64_t)bh * D + d] = fd_combine_dim(p.partials + (int64_t)bh * p.bh_stride, p.S, 2 + D, d);
}

// Threads per workgroup for a split of `split` rows at head dim d: 64 or 128 when one pass of
// that many lanes covers the split, else 256.
inline int fd_threads(int d, int split) {
  const int cl = d / 8;
  return (int64_t)split * cl <= 64 ? 64 : (int64_t)split * cl <= 128 ? 128 : 256;
}

template <int D, int KPL, int NT, bool CHUNKED>
static void fd_launch_split(const FdParams& p, bool fused, hipStream_t st) {
  if (fused) {
    const int groups = (p.B * p.H + 7) / 8;
    fd_split_kernel<D, KPL, NT, CHUNKED, true><<<dim3(8 * groups * p.S), NT, 0, st>>>(p);
  } else {
    fd_split_kernel<D, KPL, NT, CHUNKED, false><<<dim3(p.B * p.H, p.S), NT, 0, st>>>(p);
  }
}

template <int D>
static int fd_launch_d(const FdParams& p, bool fused, hipStream_t st) {
  constexpr int CL = D / 8;
  const int nt = fd_threads(D, p.split);
  if (nt == 64) {
    fd_launch_split<D, 1, 64, false>(p, fused, st);
  } else if (nt == 128) {
    fd_launch_split<D, 1, 128, false>(p, fused, st);
  } else {
    const int passes = (p.split + 256 / CL - 1) / (256 / CL);
    if (passes > kFdMaxPasses) fd_launch_split<D, kFdChunkPasses, 256, true>(p, fused, st);
    else if (passes > 8) fd_launch_split<D, 16, 256, false>(p, fused, st);
    else if (passes > 4) fd_launch_split<D, 8, 256, false>(p, fused, st);
    else if (passes > 2) fd_launch_split<D, 4, 256, false>(p, fused, st);
    else if (passes > 1) fd_launch_split<D, 2, 256, false>(p, fused, st);
    else fd_launch_split<D, 1, 256, false>(p, fused, st);
  }
  PK_LAUNCH_CHECK("flash decode split");
  if (!fused) {
    fd_combine_kernel<D><<<p.B * p.H, D < 64 ? 64 : D, 0, st>>>(p);
    PK_LAUNCH_CHECK("flash decode combine");
  }
  return PK_OK;
}

// floats between the starts of consecutive (b, h) partial regions: whole 128-byte lines
inline int64_t fd_bh_stride(int S, int D) { return ((int64_t)S * (2 + D) + 31) / 32 * 32; }

}  // namespace pk

using namespace pk;

extern "C" size_t pk_flash_decode_workspace_bytes(int B, int H, int N, int D, int split) {
  if (B < 1 || H < 1 || N < 1 || D < 1 || split < 1 || N % split) return 0;
  return kWsCounterBytes + (size_t)B * H * fd_bh_stride(N / split, D) * sizeof(float);
}

namespace {
// The splits of every (b, h) combine inside the launch when their grid fits the counters and
// the device's placement allows it (`l2`: splitk_in_l2_ok / splitk_in_l2_possible).
bool fd_fused(int B, int H, int N, int split, bool l2) {
  const int64_t bh = (int64_t)B * H, S = N / split;
  return bh <= kWsMaxTiles && 8 * ((bh + 7) / 8) * S <= 0x7fffffff && l2;
}
}  // namespace

extern "C" int pk_flash_decode_launches(int B, int H, int N, int D, int split) {
  if (B < 1 || H < 1 || N < 1 || D < 1 || split < 1 || N % split) return 0;
  return fd_fused(B, H, N, split, splitk_in_l2_possible()) ? 1 : 2;
}

extern "C" int pk_flash_decode(const void* q, int64_t sqb, int64_t sqh, const void* k,
                               int64_t skb, int64_t skh, int64_t skn, const void* v, int64_t svb,
                               int64_t svh, int64_t svn, int B, int H, int N, int D, int split,
                               float sm_scale, float* out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  PK_REQUIRE(q != nullptr && k != nullptr && v != nullptr && out != nullptr,
             "pk_flash_decode: null pointer");
  PK_REQUIRE(B >= 1 && H >= 1 && N >= 1, "pk_flash_decode: empty shape");
  PK_REQUIRE((int64_t)B * H <= 0x7fffffff / 8, "pk_flash_decode: B*H=%lld too large", (long long)B * H);
  PK_REQUIRE(D == 16 || D == 32 || D == 64 || D == 128 || D == 256,
             "pk_flash_decode: D=%d must be 16, 32, 64, 128 or 256", D);
  PK_REQUIRE(split >= 1 && N % split == 0, "pk_flash_decode: N=%d must be a multiple of split=%d", N, split);
  auto al16 = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; };
  PK_REQUIRE(al16(q) && al16(k) && al16(v) && sqb % 8 == 0 && sqh % 8 == 0 && skb % 8 == 0 &&
                 skh % 8 == 0 && skn % 8 == 0 && svb % 8 == 0 && svh % 8 == 0 && svn % 8 == 0,
             "pk_flash_decode: q/k/v need 16-byte aligned rows (strides multiples of 8)");
  const size_t need = pk_flash_decode_workspace_bytes(B, H, N, D, split);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("pk_flash_decode: workspace of %zu bytes needed (got %zu)", need, workspace_bytes);
    return PK_EWORKSPACE;
  }
  FdParams p;
  p.q = reinterpret_cast<const pk_half*>(q);
  p.sqb = sqb;
  p.sqh = sqh;
  p.k = reinterpret_cast<const pk_half*>(k);
  p.skb = skb;
  p.skh = skh;
  p.skn = skn;
  p.v = reinterpret_cast<const pk_half*>(v);
  p.svb = svb;
  p.svh = svh;
  p.svn = svn;
  p.partials = ws_partials(workspace);
  p.counters = ws_counters(workspace);
  p.out = out;
  p.B = B;
  p.H = H;
  p.N = N;
  p.split = split;
  p.S = N / split;
  p.bh_stride = fd_bh_stride(p.S, D);
  const int rg = 256 / (D / 8);
  p.nch = (split + kFdChunkPasses * rg - 1) / (kFdChunkPasses * rg);
  p.sm_scale = sm_scale;
  const bool fused = fd_fused(B, H, N, split, splitk_in_l2_ok((hipStream_t)stream));
  PK_REQUIRE(fused || p.S <= 65535, "pk_flash_decode: N/split=%d splits exceed the grid (at most 65535 "
             "when B*H > %d)", p.S, kWsMaxTiles);
  hipStream_t s = (hipStream_t)stream;
  switch (D) {
    case 16: return fd_launch_d<16>(p, fused, s);
    case 32: return fd_launch_d<32>(p, fused, s);
    case 64: return fd_launch_d<64>(p, fused, s);
    case 128: return fd_launch_d<128>(p, fused, s);
    default: return fd_launch_d<256>(p, fused, s);
  }
}
