/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle for the integer half of the per-symbol
 * step.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load this file's library, and only as a checker or as the timed CPU
 * baseline.  The product path never calls it.
 *
 * Restates, in plain C with IEEE double arithmetic and no FMA contraction
 * (built with -ffp-contract=off):
 *
 *   oracle_scale_cum   <- _scale_cum_np      src/model/arithmetic_coder_lm.py:49-64
 *                         f_i = max(1, floor(double(p_i) * 1e6 + 0.5)), C_0 = 0,
 *                         C_{i+1} = C_i + f_i, total = C_V.
 *   oracle_scale_cum_f64  the same on float64 rows
 *   oracle_wnc_encode  <- encode_with_probs  src/model/arithmetic_coder_lm.py:140-195
 *                         (+ _renorm_encode 90-112, _pack_bits 115-128)
 *   oracle_wnc_decode  <- decode_with_probs  src/model/arithmetic_coder_lm.py:198-288
 *                         (+ _bit_iter 131-137: MSB-first, zero padded)
 *
 * The coder is the 32-bit Witten-Neal-Cleary arithmetic coder (CACM 30(6),
 * 1987) with E3 "pending" bits; constants HALF = 2^31, QUARTER = 2^30.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define WNC_TOP ((uint64_t)1 << 32)
#define WNC_HALF ((uint64_t)1 << 31)
#define WNC_QUARTER ((uint64_t)1 << 30)

/* One row: probs[V] (float32) -> cum[V+1] (int64).  Returns total. */
int64_t oracle_scale_cum(const float *probs, int64_t V, int64_t *cum) {
  int64_t acc = 0;
  cum[0] = 0;
  for (int64_t i = 0; i < V; ++i) {
    double p = (double)probs[i];
    double t = p * 1000000.0; /* first rounding (numpy: p * 1_000_000.0) */
    t = t + 0.5;              /* second rounding (numpy: + 0.5) */
    double f = floor(t);
    int64_t v = (int64_t)f;
    if (v < 1) v = 1; /* np.maximum(1, ...) */
    acc += v;
    cum[i + 1] = acc;
  }
  return acc;
}

/* rows x V batch; cum is rows x (V+1). */
void oracle_scale_cum_rows(const float *probs, int64_t rows, int64_t V,
                           int64_t *cum) {
  for (int64_t r = 0; r < rows; ++r)
    oracle_scale_cum(probs + r * V, V, cum + r * (V + 1));
}

/* The same rule on float64 probabilities (the reference converts its input
 * to float64 first, arithmetic_coder_lm.py:58-60).  Here the two double
 * roundings are not exact in general. */
int64_t oracle_scale_cum_f64(const double *probs, int64_t V, int64_t *cum) {
  int64_t acc = 0;
  cum[0] = 0;
  for (int64_t i = 0; i < V; ++i) {
    double t = probs[i] * 1000000.0;
    t = t + 0.5;
    double f = floor(t);
    int64_t v = (f >= 1.0) ? (int64_t)f : 1; /* np.maximum(1, ...); NaN -> 1 */
    acc += v;
    cum[i + 1] = acc;
  }
  return acc;
}

void oracle_scale_cum_rows_f64(const double *probs, int64_t rows, int64_t V,
                               int64_t *cum) {
  for (int64_t r = 0; r < rows; ++r)
    oracle_scale_cum_f64(probs + r * V, V, cum + r * (V + 1));
}

typedef struct {
  uint8_t *bits; /* one byte per bit (0/1) */
  int64_t n, cap;
  int err;
} bitbuf;

static void bb_push(bitbuf *b, int bit) {
  if (b->n == b->cap) {
    int64_t nc = b->cap ? b->cap * 2 : 4096;
    uint8_t *p = (uint8_t *)realloc(b->bits, (size_t)nc);
    if (!p) {
      b->err = 1;
      return;
    }
    b->bits = p;
    b->cap = nc;
  }
  b->bits[b->n++] = (uint8_t)bit;
}

/*
 * Encode n symbols.  cum_rows holds n tables of V+1 int64 cumulative counts
 * (as produced by oracle_scale_cum); the total of row i is cum_rows[i*(V+1)+V].
 * Output: packed MSB-first bytes into out (capacity out_cap).  Returns the
 * number of bytes written, or -1 on overflow / bad symbol.
 */
int64_t oracle_wnc_encode(const int64_t *syms, int64_t n, const int64_t *cum_rows,
                          int64_t V, uint8_t *out, int64_t out_cap) {
  uint64_t low = 0, high = WNC_TOP - 1, pending = 0;
  bitbuf bb = {0};
  for (int64_t i = 0; i < n; ++i) {
    int64_t s = syms[i];
    if (s < 0 || s >= V) {
      free(bb.bits);
      return -1;
    }
    const int64_t *cum = cum_rows + i * (V + 1);
    uint64_t total = (uint64_t)cum[V];
    uint64_t lo_c = (uint64_t)cum[s], hi_c = (uint64_t)cum[s + 1];
    uint64_t range = high - low + 1;
    high = low + (range * hi_c) / total - 1;
    low = low + (range * lo_c) / total;
    for (;;) { /* _renorm_encode */
      if (high < WNC_HALF) {
        bb_push(&bb, 0);
        while (pending) {
          bb_push(&bb, 1);
          pending--;
        }
      } else if (low >= WNC_HALF) {
        bb_push(&bb, 1);
        while (pending) {
          bb_push(&bb, 0);
          pending--;
        }
        low -= WNC_HALF;
        high -= WNC_HALF;
      } else if (low >= WNC_QUARTER && high < 3 * WNC_QUARTER) {
        pending++;
        low -= WNC_QUARTER;
        high -= WNC_QUARTER;
      } else {
        break;
      }
      low <<= 1;
      high = (high << 1) | 1;
    }
  }
  /* flush */
  pending++;
  if (low < WNC_QUARTER) {
    bb_push(&bb, 0);
    while (pending) {
      bb_push(&bb, 1);
      pending--;
    }
  } else {
    bb_push(&bb, 1);
    while (pending) {
      bb_push(&bb, 0);
      pending--;
    }
  }
  if (bb.err) {
    free(bb.bits);
    return -1;
  }
  int64_t nbytes = (bb.n + 7) / 8;
  if (nbytes > out_cap) {
    free(bb.bits);
    return -1;
  }
  memset(out, 0, (size_t)nbytes);
  for (int64_t i = 0; i < bb.n; ++i)
    if (bb.bits[i]) out[i >> 3] |= (uint8_t)(0x80u >> (i & 7));
  free(bb.bits);
  return nbytes;
}

static int read_bit(const uint8_t *data, int64_t nbytes, int64_t *pos) {
  int64_t i = (*pos)++;
  if ((i >> 3) >= nbytes) return 0; /* zero padding past the end */
  return (data[i >> 3] >> (7 - (i & 7))) & 1;
}

/*
 * Decode n symbols.  The caller provides all n tables up front (teacher-forced
 * rows, as the reference tests do); returns 0 on success.
 */
int oracle_wnc_decode(const uint8_t *data, int64_t nbytes, int64_t n,
                      const int64_t *cum_rows, int64_t V, int64_t *out_syms) {
  uint64_t low = 0, high = WNC_TOP - 1, value = 0;
  int64_t bitpos = 0;
  for (int k = 0; k < 32; ++k) value = (value << 1) | (uint64_t)read_bit(data, nbytes, &bitpos);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t *cum = cum_rows + i * (V + 1);
    uint64_t total = (uint64_t)cum[V];
    uint64_t range = high - low + 1;
    uint64_t offset = ((value - low + 1) * total - 1) / range;
    /* largest s with cum[s] <= offset (np.searchsorted(cum, offset, 'right') - 1) */
    int64_t lo = 0, hi = V + 1;
    while (lo < hi) {
      int64_t mid = (lo + hi) / 2;
      if ((uint64_t)cum[mid] <= offset)
        lo = mid + 1;
      else
        hi = mid;
    }
    int64_t s = lo - 1;
    if (s < 0) s = 0;
    if (s > V - 1) s = V - 1;
    out_syms[i] = s;
    uint64_t lo_c = (uint64_t)cum[s], hi_c = (uint64_t)cum[s + 1];
    high = low + (range * hi_c) / total - 1;
    low = low + (range * lo_c) / total;
    for (;;) {
      if (high < WNC_HALF) {
      } else if (low >= WNC_HALF) {
        low -= WNC_HALF;
        high -= WNC_HALF;
        value -= WNC_HALF;
      } else if (low >= WNC_QUARTER && high < 3 * WNC_QUARTER) {
        low -= WNC_QUARTER;
        high -= WNC_QUARTER;
        value -= WNC_QUARTER;
      } else {
        break;
      }
      low <<= 1;
      high = (high << 1) | 1;
      value = (value << 1) | (uint64_t)read_bit(data, nbytes, &bitpos);
    }
  }
  return 0;
}
