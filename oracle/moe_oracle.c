/*
 * moe_oracle.c -- plain-C restatement of the reference's MoE dispatch math.
 *
 * TEST INFRASTRUCTURE ONLY: built into oracle/liboracle.so by oracle/oracle_c.py
 * and called from tests/ as the checker.  Compiled with -ffp-contract=off so
 * every fp32 operation rounds exactly as written.  Paths are relative to the
 * reference repository.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* fp32 -> bf16 bits, round to nearest even (case25...py:56-66); NaN -> 0x7FC0. */
uint16_t oracle_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/*
 * Row-id map (kernel_cases/case12_moe_row_id_map_pass2.py:43-50): expert by
 * expert, tokens in ascending order get consecutive rows; unselected -> -1.
 * Writes the token-major map row_tm [T*E] and offsets [E+1].
 */
void oracle_row_id_map(const uint8_t *mask, int64_t T, int64_t E, int64_t *row_tm, int64_t *offsets) {
  int64_t next = 0;
  for (int64_t e = 0; e < E; ++e) {
    offsets[e] = next;
    for (int64_t t = 0; t < T; ++t) {
      if (mask[t * E + e]) {
        row_tm[t * E + e] = next++;
      } else {
        row_tm[t * E + e] = -1;
      }
    }
  }
  offsets[E] = next;
}

/*
 * Permute (case17...py:58-71; case21/22/30 for the expert-major layout):
 * out[map(t,e)] = x[t] (row_bytes bytes), pp[map(t,e)] = probs[t,e];
 * rows never written are zero.  map is int64, layout 0 = [T,E], 1 = [E,T].
 * Entries >= num_out are skipped.
 */
void oracle_permute(const uint8_t *x, int64_t T, int64_t row_bytes, const int64_t *map, int layout, int64_t E,
                    const float *probs, uint8_t *out, float *pp, int64_t num_out) {
  memset(out, 0, (size_t)(num_out * row_bytes));
  if (pp) memset(pp, 0, (size_t)num_out * sizeof(float));
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t e = 0; e < E; ++e) {
      const int64_t d = layout == 0 ? map[t * E + e] : map[e * T + t];
      if (d < 0 || d >= num_out) continue;
      memcpy(out + d * row_bytes, x + t * row_bytes, (size_t)row_bytes);
      if (pp && probs) pp[d] = probs[t * E + e];
    }
  }
}

/*
 * Unpermute (case15...py:58-64, case24...py:45-68) and its merge form:
 * acc[t] = 0; for e ascending with map(t,e) in [0,R): acc += [w *] float(pin[map]);
 * out[t] = bf16_rne(acc).  probs (nullable) is [T,E].  acc_out (nullable) gets acc.
 */
void oracle_unpermute(const uint16_t *pin, int64_t R, int64_t H, const int64_t *map, int layout, int64_t E,
                      int64_t T, const float *probs, uint16_t *out, float *acc_out) {
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t h = 0; h < H; ++h) {
      float acc = 0.0f;
      for (int64_t e = 0; e < E; ++e) {
        const int64_t s = layout == 0 ? map[t * E + e] : map[e * T + t];
        if (s < 0 || s >= R) continue;
        const float v = bf16_to_f32(pin[s * H + h]);
        if (probs) {
          const float p = probs[t * E + e] * v;
          acc = acc + p;
        } else {
          acc = acc + v;
        }
      }
      out[t * H + h] = oracle_bf16_rne(acc);
      if (acc_out) acc_out[t * H + h] = acc;
    }
  }
}

/* Permute backward prob-gradient gather (case18...py:74-77): dprobs[t,e] = dpp[map] or 0. */
void oracle_prob_gather(const float *dpp, int64_t R, const int64_t *map, int layout, int64_t E, int64_t T,
                        float *dprobs) {
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t e = 0; e < E; ++e) {
      const int64_t s = layout == 0 ? map[t * E + e] : map[e * T + t];
      dprobs[t * E + e] = (s >= 0 && s < R) ? dpp[s] : 0.0f;
    }
  }
}

/* True when a ranks strictly before b in a stable descending sort (NaN largest, -0 == +0). */
static int ranks_before(float a, int64_t ia, float b, int64_t ib) {
  const int na = isnan(a), nb = isnan(b);
  if (na || nb) {
    if (na && nb) return ia < ib;
    return na;
  }
  if (a > b) return 1;
  if (a < b) return 0;
  return ia < ib;
}

/*
 * Top-k (case23...py:47-62): the first k of a stable descending sort, by k
 * passes of selection over each row.
 */
void oracle_topk(const float *x, int64_t T, int64_t E, int64_t k, float *values, int64_t *indices) {
  for (int64_t t = 0; t < T; ++t) {
    const float *row = x + t * E;
    for (int64_t j = 0; j < k; ++j) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        int taken = 0;
        for (int64_t q = 0; q < j; ++q) taken |= indices[t * k + q] == e;
        if (taken) continue;
        if (best < 0 || ranks_before(row[e], e, row[best], best)) best = e;
      }
      indices[t * k + j] = best;
      values[t * k + j] = row[best];
    }
  }
}

/* Row gather (case06...py:38-40): out[i] = src[index[i]] (row_bytes bytes each). */
void oracle_index_select(const uint8_t *src, int64_t src_rows, int64_t row_bytes, const int64_t *index,
                         int64_t n, uint8_t *out) {
  for (int64_t i = 0; i < n; ++i) {
    const int64_t s = index[i];
    if (s >= 0 && s < src_rows) {
      memcpy(out + i * row_bytes, src + s * row_bytes, (size_t)row_bytes);
    } else {
      memset(out + i * row_bytes, 0, (size_t)row_bytes);
    }
  }
}
