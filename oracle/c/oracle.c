/* C restatement of the reference's 8-bit split-K decode and of MLX's affine
 * 8-bit quantizer -- TEST INFRASTRUCTURE (the checker and the timed CPU
 * baseline), never the product path.
 *
 * orc_attend_q8  follows locals/qkv.py:213-249 (launcher: block of 1,024 keys up
 *                to 16k, 2,048 beyond, qkv.py:232), pass 1 qkv.py:30-87 (per
 *                (row, kv head, block): a running softmax per query head over
 *                the block's keys, q pre-scaled, dequantization scale*code+bias
 *                in fp32) and pass 2 qkv.py:179-208 (log-sum-exp join of the
 *                blocks with the head's sink in the denominator).  fp32
 *                throughout, OpenMP over (row, kv head, block) like the
 *                reference's threadgroups.
 * orc_quantize   MLX affine quantize, bits 8 (mx.quantize as called at
 *                qkv.py:322-323): per group min/max, scale, edge, q0, codes.
 *                Returns fp32 scale/bias (the caller casts to the 16-bit dtype,
 *                round to nearest even).  round_mode 0 = half away from zero
 *                (roundf, Metal round), 1 = half to even (rintf).
 *
 * orc_sdpa       MLX scaled_dot_product_attention as the reference's multi-query
 *                variants call it (qkv.attention's prompt branch over the
 *                dequantized cache, locals/qkv.py:270-272 -> fuse.attend_few,
 *                locals/fuse.py:131-144; tree verification, locals/treedec.py:
 *                56-79): K/V given as fp32 values (the caller dequantizes and
 *                rounds them to the activation dtype), masks: causal aligned to
 *                the last key (fuse.py:131-137), tree (prefix visible, new keys by
 *                ancestor bits), dense, sliding window, left padding; the sink a
 *                logit in the denominator only.  Scores are fp32 dot products;
 *                the softmax sums and the P V accumulation are double.  OpenMP
 *                over (row, kv head, block of 16 queries).
 * Build: oracle/Makefile (gcc -O2 -fopenmp, no fast-math: divisions stay
 * correctly rounded and nothing is contracted).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float rnd(float x, int mode) { return mode ? rintf(x) : roundf(x); }

void orc_quantize(const float *w, int64_t rows, int D, int group, int round_mode,
                  uint8_t *codes, float *scales, float *biases) {
  const int ng = D / group;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    for (int g = 0; g < ng; g++) {
      const float *x = w + r * D + g * group;
      float w_max = -INFINITY, w_min = INFINITY;
      for (int i = 0; i < group; i++) {
        w_max = fmaxf(w_max, x[i]);
        w_min = fminf(w_min, x[i]);
      }
      const float n_bins = 255.0f, eps = 1e-7f;
      float scale = fmaxf((w_max - w_min) / n_bins, eps);
      const int side = fabsf(w_min) > fabsf(w_max);
      scale = side ? scale : -scale;
      const float edge = side ? w_min : w_max;
      const float q0 = rnd(edge / scale, round_mode);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      for (int i = 0; i < group; i++) {
        float c = rnd((x[i] - bias) / scale, round_mode);
        c = fminf(fmaxf(c, 0.0f), n_bins);
        codes[r * D + g * group + i] = (uint8_t)c;
      }
      scales[r * ng + g] = scale;
      biases[r * ng + g] = bias;
    }
  }
}

/* q (B,H,HD) fp32 values; kw/vw (B,KVH,cap,HD/4) uint32 words; ks/kb/vs/vb
 * (B,KVH,cap,HD/64) fp32 values of the 16-bit scales/biases; start (B,);
 * sinks (H,) or NULL; out (B,H,HD).  block = 0 picks the reference's size. */
int orc_attend_q8(const float *q, const uint32_t *kw, const float *ks, const float *kb,
                  const uint32_t *vw, const float *vs, const float *vb, const int32_t *start,
                  const float *sinks, float scale, int B, int H, int KVH, int HD, int cap, int n,
                  int block, float *out) {
  if (H % KVH || HD % 64 || n > cap) return -1;
  const int G = H / KVH, WPR = HD / 4, GPR = HD / 64;
  if (!block) block = n <= 16384 ? 1024 : 2048;
  const int nb = n > 0 ? (n + block - 1) / block : 1;
  float *pm = malloc(sizeof(float) * (size_t)B * H * nb);
  float *pl = malloc(sizeof(float) * (size_t)B * H * nb);
  float *po = malloc(sizeof(float) * (size_t)B * H * nb * HD);
  if (!pm || !pl || !po) { free(pm); free(pl); free(po); return -2; }
  /* pass 1: one part per (row, head, block) */
#pragma omp parallel for collapse(3) schedule(dynamic, 1)
  for (int b = 0; b < B; b++)
    for (int h = 0; h < KVH; h++)
      for (int j = 0; j < nb; j++) {
        const int s0 = start[b] > 0 ? start[b] : 0;
        const int lo = j * block > s0 ? j * block : s0;
        const int hi = (j + 1) * block < n ? (j + 1) * block : n;
        float *qs = malloc(sizeof(float) * (size_t)G * HD);
        float *m = malloc(sizeof(float) * (size_t)G), *l = malloc(sizeof(float) * (size_t)G);
        float *o = malloc(sizeof(float) * (size_t)G * HD);
        float *kv = malloc(sizeof(float) * 2 * (size_t)HD);
        for (int g = 0; g < G; g++) {
          for (int d = 0; d < HD; d++) qs[g * HD + d] = q[((size_t)b * H + h * G + g) * HD + d] * scale;
          m[g] = -INFINITY;
          l[g] = 0.0f;
        }
        memset(o, 0, sizeof(float) * (size_t)G * HD);
        const size_t row0 = ((size_t)b * KVH + h) * cap;
        for (int t = lo; t < hi; t++) {
          const size_t r = row0 + t;
          for (int d = 0; d < HD; d++) {
            const int grp = d / 64;
            const uint32_t kc = (kw[r * WPR + d / 4] >> (8 * (d % 4))) & 0xffu;
            const uint32_t vc = (vw[r * WPR + d / 4] >> (8 * (d % 4))) & 0xffu;
            kv[d] = ks[r * GPR + grp] * (float)kc + kb[r * GPR + grp];
            kv[HD + d] = vs[r * GPR + grp] * (float)vc + vb[r * GPR + grp];
          }
          for (int g = 0; g < G; g++) {
            float sc = 0.0f;
            for (int d = 0; d < HD; d++) sc += qs[g * HD + d] * kv[d];
            const float m2 = fmaxf(m[g], sc);
            const float corr = expf(m[g] - m2), p = expf(sc - m2);
            l[g] = l[g] * corr + p;
            for (int d = 0; d < HD; d++) o[g * HD + d] = o[g * HD + d] * corr + p * kv[HD + d];
            m[g] = m2;
          }
        }
        for (int g = 0; g < G; g++) {
          const size_t part = ((size_t)b * H + h * G + g) * nb + j;
          pm[part] = m[g];
          pl[part] = l[g];
          memcpy(po + part * HD, o + (size_t)g * HD, sizeof(float) * HD);
        }
        free(qs);
        free(m);
        free(l);
        free(o);
        free(kv);
      }
  /* pass 2: join the blocks with the sink */
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; b++)
    for (int hh = 0; hh < H; hh++) {
      const size_t sg = (size_t)b * H + hh;
      const float sink = sinks ? sinks[hh] : -INFINITY;
      float M = sink;
      for (int j = 0; j < nb; j++) M = fmaxf(M, pm[sg * nb + j]);
      float *dst = out + sg * HD;
      if (M == -INFINITY) {
        memset(dst, 0, sizeof(float) * HD);
        continue;
      }
      float L = sinks ? expf(sink - M) : 0.0f;
      for (int d = 0; d < HD; d++) dst[d] = 0.0f;
      for (int j = 0; j < nb; j++) {
        const float mj = pm[sg * nb + j];
        const float w = mj == -INFINITY ? 0.0f : expf(mj - M);
        L += pl[sg * nb + j] * w;
        for (int d = 0; d < HD; d++) dst[d] += po[(sg * nb + j) * HD + d] * w;
      }
      for (int d = 0; d < HD; d++) dst[d] /= L;
    }
  free(pm);
  free(pl);
  free(po);
  return 0;
}

/* q (B,H,L,D); k, v (B,KVH,cap,D) fp32 values; keys [0, N) of each buffer row.
 * mask_kind 0 none, 1 causal (query i sees key j <= N - L + i), 2 tree (key
 * j < N - L for all; key N - L + d iff bit d of tree[b*L + i]), 3 dense
 * (dense[(b*L + i)*N + j] != 0, shared by the heads), 4 window (N - L + i -
 * window < j <= N - L + i).  start (B,) or NULL hides keys before start[b].
 * sinks (H,) or NULL.  out (B,H,L,D); a query with no visible key and no sink
 * gives 0. */
int orc_sdpa(const float *q, const float *k, const float *v, const int32_t *start, int mask_kind,
             const uint64_t *tree, const uint8_t *dense, int window, const float *sinks, float scale, int B,
             int H, int KVH, int L, int N, int D, int cap, float *out) {
  if (H % KVH || N > cap || L > N || (mask_kind == 2 && L > 64) || mask_kind < 0 || mask_kind > 4) return -1;
  const int G = H / KVH, QB = 16;
  const int nqb = (L + QB - 1) / QB;
  const int off = N - L;
  int fail = 0;
#pragma omp parallel for collapse(3) schedule(dynamic, 1)
  for (int b = 0; b < B; b++)
    for (int h = 0; h < KVH; h++)
      for (int qb = 0; qb < nqb; qb++) {
        const int i0 = qb * QB, i1 = i0 + QB < L ? i0 + QB : L;
        const int R = (i1 - i0) * G; /* rows: (query i, head g) */
        float *qs = malloc(sizeof(float) * (size_t)R * D); /* transposed: qs[d * R + r] */
        float *acc = malloc(sizeof(float) * (size_t)R);
        float *S = malloc(sizeof(float) * (size_t)R * N);
        double *o = malloc(sizeof(double) * (size_t)R * D);
        double *den = malloc(sizeof(double) * (size_t)R);
        float *M = malloc(sizeof(float) * (size_t)R);
        if (!qs || !acc || !S || !o || !den || !M) {
#pragma omp atomic write
          fail = 1;
          free(qs); free(acc); free(S); free(o); free(den); free(M);
          continue;
        }
        for (int i = i0; i < i1; i++)
          for (int g = 0; g < G; g++) {
            const int r = (i - i0) * G + g;
            const float *src = q + (((size_t)b * H + h * G + g) * L + i) * D;
            for (int d = 0; d < D; d++) qs[(size_t)d * R + r] = src[d];
          }
        const size_t kv0 = ((size_t)b * KVH + h) * cap;
        const int s0 = start && start[b] > 0 ? start[b] : 0;
        /* scores: key j against every row; each row's sum runs over the dims in order, the rows side by side */
        for (int j = 0; j < N; j++) {
          const float *kj = k + (kv0 + j) * D;
          for (int r = 0; r < R; r++) acc[r] = 0.0f;
          for (int d = 0; d < D; d++) {
            const float kd = kj[d];
            const float *qd = qs + (size_t)d * R;
            for (int r = 0; r < R; r++) acc[r] += qd[r] * kd;
          }
          for (int r = 0; r < R; r++) {
            const int i = i0 + r / G;
            int vis = j >= s0;
            if (mask_kind == 1) vis = vis && j <= off + i;
            else if (mask_kind == 2) vis = vis && (j < off || ((tree[(size_t)b * L + i] >> (j - off)) & 1u));
            else if (mask_kind == 3) vis = vis && dense[((size_t)b * L + i) * N + j];
            else if (mask_kind == 4) vis = vis && j <= off + i && j > off + i - window;
            S[(size_t)r * N + j] = vis ? acc[r] * scale : -INFINITY;
          }
        }
        for (int r = 0; r < R; r++) {
          const int g = r % G;
          const float sink = sinks ? sinks[h * G + g] : -INFINITY;
          float m = sink;
          for (int j = 0; j < N; j++) m = fmaxf(m, S[(size_t)r * N + j]);
          M[r] = m;
          den[r] = (m == -INFINITY || !sinks) ? 0.0 : exp((double)sink - (double)m);
          for (int d = 0; d < D; d++) o[(size_t)r * D + d] = 0.0;
        }
        for (int j = 0; j < N; j++) {
          const float *vj = v + (kv0 + j) * D;
          for (int r = 0; r < R; r++) {
            const float sj = S[(size_t)r * N + j];
            if (sj == -INFINITY) continue;
            const double p = exp((double)sj - (double)M[r]);
            den[r] += p;
            double *orow = o + (size_t)r * D;
            for (int d = 0; d < D; d++) orow[d] += p * (double)vj[d];
          }
        }
        for (int i = i0; i < i1; i++)
          for (int g = 0; g < G; g++) {
            const int r = (i - i0) * G + g;
            float *dst = out + (((size_t)b * H + h * G + g) * L + i) * D;
            for (int d = 0; d < D; d++) dst[d] = den[r] > 0.0 ? (float)(o[(size_t)r * D + d] / den[r]) : 0.0f;
          }
        free(qs); free(acc); free(S); free(o); free(den); free(M);
      }
  return fail ? -2 : 0;
}
