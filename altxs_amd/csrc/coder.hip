// Range coder on the device: the 32-bit Witten-Neal-Cleary arithmetic coder
// with E3 ("pending") bits that the reference runs on the host
// (src/model/arithmetic_coder_lm.py:90-288) and, one thread and one int64 per
// bit, on the GPU (src/xsa_ttt/gpu_ac.py:84-218, 397-479).
//
// Here every segment is its own stream with its state in device memory
// (AltxsCoderState), so B segments code in parallel, and the coder reads the
// integer CDF rows the step already produced (uint32 cum[V+1], total =
// cum[V]) -- no per-symbol rescaling.  Bits are packed MSB-first into bytes
// on the device (the reference's _pack_bits layout); a stream's bytes go to
// buf + b * stride.
//
//   encode: one lane per stream, W symbols in order; the three table reads
//           of a symbol do not depend on the coder state, so they are issued
//           ahead of the arithmetic;
//   decode: one wave per stream; the symbol search over cum (largest s with
//           cum[s] <= offset) is a 64-ary search: each round the 64 lanes
//           sample the current range and a ballot narrows it 64-fold, so
//           V = 65536 takes three rounds of loads instead of 17 dependent ones.
//           The decoded symbol is written where the next step reads its token.
#include "common.h"

namespace {

constexpr uint64_t TOP = 1ull << 32, HALF = 1ull << 31, QUARTER = 1ull << 30;

// A symbol's table entries the coder can use: non-empty, inside [0, tot],
// tot at most QUARTER (the step's tables total about 1e6 + V).
__device__ __forceinline__ bool table_ok(uint64_t lo, uint64_t hi, uint64_t tot) {
  return tot > 0 && tot <= QUARTER && lo < hi && hi <= tot;
}

struct Enc {
  uint64_t low, high, pending;
  int64_t nbits;
  uint32_t cur;  // bits of the byte being filled (nbits % 8 of them, MSB first)
  uint8_t* out;
  int64_t cap;
  int32_t err;

  __device__ void put(int bit) {
    cur = (cur << 1) | (uint32_t)bit;
    ++nbits;
    if ((nbits & 7) == 0) {
      const int64_t i = (nbits >> 3) - 1;
      if (i < cap) out[i] = (uint8_t)cur;
      else err |= 1;
      cur = 0;
    }
  }
  __device__ void put_run(int bit) {  // bit, then the pending bits inverted
    put(bit);
    for (; pending; --pending) put(bit ^ 1);
  }
};

__device__ __forceinline__ void load_enc(Enc& e, const AltxsCoderState& s, uint8_t* out, int64_t cap) {
  e.low = s.low; e.high = s.high; e.pending = s.pending; e.nbits = s.nbits;
  e.cur = (uint32_t)s.partial; e.out = out; e.cap = cap; e.err = 0;
}
__device__ __forceinline__ void store_enc(const Enc& e, AltxsCoderState& s) {
  s.low = e.low; s.high = e.high; s.pending = e.pending; s.nbits = e.nbits;
  s.partial = e.cur;
  s.err |= e.err;
}

__global__ __launch_bounds__(64) void encode_kernel(AltxsCoderState* __restrict__ st, int n, int W,
                                                    const int32_t* __restrict__ syms,
                                                    const uint32_t* __restrict__ cum, int V,
                                                    uint8_t* buf, int64_t stride) {
  const int b = blockIdx.x * 64 + threadIdx.x;
  if (b >= n) return;
  Enc e;
  load_enc(e, st[b], buf + (int64_t)b * stride, stride);
  const int64_t row0 = (int64_t)b * W;
  // operands of symbol t + 1 are loaded while symbol t is coded
  auto fetch = [&](int t, uint32_t& lo, uint32_t& hi, uint32_t& tot, int& bad) {
    const int s = syms[row0 + t];
    const uint32_t* c = cum + (row0 + t) * (int64_t)(V + 1);
    bad = s < 0 || s >= V;
    const int sc = bad ? 0 : s;
    lo = c[sc];
    hi = c[sc + 1];
    tot = c[V];
  };
  uint32_t lo, hi, tot;
  int bad;
  if (W > 0) fetch(0, lo, hi, tot, bad);
  for (int t = 0; t < W; ++t) {
    uint32_t nlo = 0, nhi = 0, ntot = 1;
    int nbad = 0;
    if (t + 1 < W) fetch(t + 1, nlo, nhi, ntot, nbad);
    // hi <= tot <= QUARTER < range keeps the new interval non-empty and
    // inside the old one, so each renormalisation round doubles the range
    // and the loop ends within 32 rounds (the cap only guards bad state)
    if (bad || !table_ok(lo, hi, tot) || e.high < e.low || e.high >= TOP) {
      e.err |= 2;
    } else {
      const uint64_t range = e.high - e.low + 1;
      e.high = e.low + (range * hi) / tot - 1;
      e.low = e.low + (range * lo) / tot;
      for (int guard = 0; guard < 64; ++guard) {
        if (e.high < HALF) {
          e.put_run(0);
        } else if (e.low >= HALF) {
          e.put_run(1);
          e.low -= HALF;
          e.high -= HALF;
        } else if (e.low >= QUARTER && e.high < 3 * QUARTER) {
          ++e.pending;
          e.low -= QUARTER;
          e.high -= QUARTER;
        } else {
          break;
        }
        e.low <<= 1;
        e.high = (e.high << 1) | 1;
      }
    }
    lo = nlo; hi = nhi; tot = ntot; bad = nbad;
  }
  store_enc(e, st[b]);
}

__global__ __launch_bounds__(64) void finish_kernel(AltxsCoderState* __restrict__ st, int n,
                                                    uint8_t* buf, int64_t stride) {
  const int b = blockIdx.x * 64 + threadIdx.x;
  if (b >= n) return;
  Enc e;
  load_enc(e, st[b], buf + (int64_t)b * stride, stride);
  ++e.pending;
  e.put_run(e.low < QUARTER ? 0 : 1);
  const int r = (int)(e.nbits & 7);
  if (r) {  // last partial byte, zero padded
    const int64_t i = e.nbits >> 3;
    if (i < e.cap) e.out[i] = (uint8_t)(e.cur << (8 - r));
    else e.err |= 1;
  }
  store_enc(e, st[b]);
  st[b].nbytes = (e.nbits + 7) >> 3;
}

__global__ __launch_bounds__(64) void init_kernel(AltxsCoderState* __restrict__ st, int n) {
  const int b = blockIdx.x * 64 + threadIdx.x;
  if (b >= n) return;
  AltxsCoderState& s = st[b];
  s.low = 0; s.high = TOP - 1; s.pending = 0; s.value = 0; s.nbits = 0; s.nbytes = 0;
  s.partial = 0; s.err = 0;
}

__device__ __forceinline__ int read_bit(const uint8_t* in, int64_t nbytes, int64_t pos) {
  if (pos < 0 || (pos >> 3) >= nbytes) return 0;  // zero padding past the end
  return (in[pos >> 3] >> (7 - (pos & 7))) & 1;
}

__global__ __launch_bounds__(64) void seed_kernel(AltxsCoderState* __restrict__ st, int n,
                                                  const uint8_t* buf, int64_t stride,
                                                  const int64_t* nbytes) {
  const int b = blockIdx.x * 64 + threadIdx.x;
  if (b >= n) return;
  const uint8_t* in = buf + (int64_t)b * stride;
  const int64_t want = nbytes[b];
  const int64_t nb = want < 0 ? 0 : want > stride ? stride : want;  // reads stay in the row
  uint64_t v = 0;
  for (int k = 0; k < 32; ++k) v = (v << 1) | (uint64_t)read_bit(in, nb, k);
  AltxsCoderState& s = st[b];
  s.low = 0; s.high = TOP - 1; s.pending = 0; s.value = v; s.nbits = 32; s.partial = 0;
  s.nbytes = nb; s.err = nb == want ? 0 : 1;
}

// One wave per stream: decode one symbol from cum row b (V + 1 entries).
__global__ __launch_bounds__(64) void decode_kernel(AltxsCoderState* __restrict__ st, int n,
                                                    const uint32_t* __restrict__ cum, int V,
                                                    const uint8_t* buf, int64_t stride,
                                                    int32_t* out, int64_t out_stride) {
  const int b = blockIdx.x;
  if (b >= n) return;
  const int lane = threadIdx.x;
  const uint32_t* c = cum + (int64_t)b * (V + 1);
  AltxsCoderState& s = st[b];
  const uint64_t low = s.low, high = s.high, value = s.value;
  const uint64_t total = c[V];
  const uint64_t range = high - low + 1;
  const bool state_ok = low <= high && high < TOP && total > 0 && total <= QUARTER;
  const uint64_t offset = state_ok ? ((value - low + 1) * total - 1) / range : 0;
  // largest idx in [0, V] with c[idx] <= offset: 64-ary search over [lo, lo + span)
  int lo = 0, span = V + 1;
  while (span > 1) {
    const int step = (span + 63) / 64;
    const int idx = lo + lane * step;
    const bool le = lane * step < span && (uint64_t)c[idx] <= offset;
    const uint64_t mask = __ballot(le);
    const int cnt = __popcll(mask);  // c is increasing: the lanes <= offset are a prefix
    if (cnt == 0) break;             // offset below c[0] (= 0): cannot happen for valid tables
    lo += (cnt - 1) * step;
    const int rest = span - (cnt - 1) * step;
    span = step < rest ? step : rest;
  }
  int sym = lo < V ? lo : V - 1;
  if (lane == 0) {
    const uint8_t* in = buf + (int64_t)b * stride;
    const int64_t nb = s.nbytes < 0 ? 0 : s.nbytes > stride ? stride : s.nbytes;
    int64_t pos = s.nbits;
    uint64_t lw = low, hg = high, vl = value;
    int32_t err = 0;
    const uint64_t lo_c = c[sym], hi_c = c[sym + 1];
    // a valid table and state give a non-empty interval inside [low, high]
    // (as in the encoder); anything else is flagged and leaves the state be
    const bool ok = state_ok && table_ok(lo_c, hi_c, total);
    if (ok) {
      hg = lw + (range * hi_c) / total - 1;
      lw = lw + (range * lo_c) / total;
    } else {
      err |= 2;
    }
    for (int guard = 0; ok && guard < 64; ++guard) {
      if (hg < HALF) {
      } else if (lw >= HALF) {
        lw -= HALF; hg -= HALF; vl -= HALF;
      } else if (lw >= QUARTER && hg < 3 * QUARTER) {
        lw -= QUARTER; hg -= QUARTER; vl -= QUARTER;
      } else {
        break;
      }
      lw <<= 1;
      hg = (hg << 1) | 1;
      vl = (vl << 1) | (uint64_t)read_bit(in, nb, pos++);
    }
    s.low = lw; s.high = hg; s.value = vl; s.nbits = pos;
    s.err |= err;
    out[(int64_t)b * out_stride] = sym;
  }
}

}  // namespace

extern "C" int32_t altxs_range_init(AltxsCoderState* st, int32_t n, altxs_stream_t stream) {
  ALTXS_REQUIRE(st && n >= 0, "altxs_range_init: bad arguments");
  if (n == 0) return ALTXS_OK;
  hipLaunchKernelGGL(init_kernel, dim3((n + 63) / 64), dim3(64), 0, (hipStream_t)stream, st, n);
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}

extern "C" int32_t altxs_range_encode(AltxsCoderState* st, int32_t n, int32_t W, const int32_t* syms,
                                      const uint32_t* cum, int32_t V, uint8_t* buf, int64_t stride,
                                      altxs_stream_t stream) {
  ALTXS_REQUIRE(st && syms && cum && buf && n >= 0 && W >= 0 && V >= 2 && V <= (1 << 20) &&
                    stride > 0,
                "altxs_range_encode: bad arguments");
  if (n == 0 || W == 0) return ALTXS_OK;
  hipLaunchKernelGGL(encode_kernel, dim3((n + 63) / 64), dim3(64), 0, (hipStream_t)stream, st, n, W,
                     syms, cum, V, buf, stride);
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}

extern "C" int32_t altxs_range_finish(AltxsCoderState* st, int32_t n, uint8_t* buf, int64_t stride,
                                      altxs_stream_t stream) {
  ALTXS_REQUIRE(st && buf && n >= 0 && stride > 0, "altxs_range_finish: bad arguments");
  if (n == 0) return ALTXS_OK;
  hipLaunchKernelGGL(finish_kernel, dim3((n + 63) / 64), dim3(64), 0, (hipStream_t)stream, st, n, buf,
                     stride);
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}

extern "C" int32_t altxs_range_seed(AltxsCoderState* st, int32_t n, const uint8_t* buf,
                                    int64_t stride, const int64_t* nbytes, altxs_stream_t stream) {
  ALTXS_REQUIRE(st && buf && nbytes && n >= 0 && stride > 0, "altxs_range_seed: bad arguments");
  if (n == 0) return ALTXS_OK;
  hipLaunchKernelGGL(seed_kernel, dim3((n + 63) / 64), dim3(64), 0, (hipStream_t)stream, st, n, buf,
                     stride, nbytes);
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}

extern "C" int32_t altxs_range_decode(AltxsCoderState* st, int32_t n, const uint32_t* cum, int32_t V,
                                      const uint8_t* buf, int64_t stride, int32_t* out,
                                      int64_t out_stride, altxs_stream_t stream) {
  ALTXS_REQUIRE(st && cum && buf && out && n >= 0 && V >= 2 && V <= (1 << 20) && stride > 0 &&
                    out_stride >= 1,
                "altxs_range_decode: bad arguments");
  if (n == 0) return ALTXS_OK;
  hipLaunchKernelGGL(decode_kernel, dim3(n), dim3(64), 0, (hipStream_t)stream, st, n, cum, V, buf,
                     stride, out, out_stride);
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}
