/*
 * TEST INFRASTRUCTURE ONLY. CPU restatement of deformops' multi-scale deformable
 * attention (MSDA), forward and backward, used by tests/, bench.py's CPU baseline
 * and __graft_entry__.smoke() as the checker of the HIP kernels. Nothing in the
 * product path links or calls it.
 *
 * Algorithm (reference sources/deformops/backends/eager/msda_pytorch.py:23-112):
 *   x = loc_x * W - 0.5, y = loc_y * H - 0.5                     (:66-67)
 *   x0 = floor(x), x1 = x0 + 1, dx = x - x0 (same for y)           (:69-75)
 *   corner (yi, xi) counts only if 0 <= xi < W and 0 <= yi < H     (:77-80)
 *   bilinear weights (1-dx)(1-dy), dx(1-dy), (1-dx)dy, dx*dy        (:103-107)
 *   out[b,q,h,:] = sum_{l,p} attn * sum_c w_c * value[b, start_l + yi*W + xi, h, :]
 *                                                                  (:109-112)
 * A sample with a coordinate outside -1 <= pixel < size, or NaN, is skipped, as
 * the reference CUDA kernel does (backends/cuda/include/msda_forward.cuh:100-103);
 * for finite in-range input this is the eager result. The softmax method
 * normalizes the weights over the L * P points of each (b, q, h), out-of-range
 * samples included (registry/msda.py:160-182; msda_forward.cuh:92-99).
 *
 * The pixel map is rounded in float32 when pixel_f32 != 0, as the reference does
 * for float32/float16/bfloat16 inputs (its eager path in the input dtype, its
 * kernels in an fp32 accumulator), so a location on a pixel boundary lands in the
 * same cell as on the GPU. Everything else is float64.
 *
 * Backward: the gradients of the forward above (torch autograd of the eager path
 * in the reference), written out:
 *   G_c        = sum_d grad_out[d] * value_c[d]        (corner c in bounds)
 *   grad_value[c, d] += a * w_c * grad_out[d]
 *   dL/da      = sum_c w_c G_c
 *   dL/dloc_x  = a * W * ((1-dy)(G01-G00) + dy(G11-G10))
 *   dL/dloc_y  = a * H * ((1-dx)(G10-G00) + dx(G11-G01))
 *   softmax:   dL/dlogit_j = p_j (dL/dp_j - sum_i p_i dL/dp_i)
 * Parity of this file is pinned in tests/test_oracle.py against
 * torch.nn.functional.grid_sample (the reference's own definition,
 * backends/reference/msda.py:58-97) and its autograd, against a torch restatement
 * of the eager path and its autograd, against brute-force loops and closed forms.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  int64_t h, w, start;
  int ok;
} level_t;

typedef struct {
  int in;
  double dx, dy;
  int64_t pos[4];  /* positions of the 4 corners on the S axis */
  int mask[4];     /* corner inside the level */
  double w[4];     /* bilinear weights, zero for corners outside */
} geom_t;

static void geometry(double lx, double ly, const level_t* lv, int pixel_f32, geom_t* g) {
  double x, y;
  if (pixel_f32) {
    volatile float fx = (float)lx * (float)lv->w;
    volatile float fy = (float)ly * (float)lv->h;
    fx = fx - 0.5f;
    fy = fy - 0.5f;
    x = fx;
    y = fy;
  } else {
    volatile double px = lx * (double)lv->w;
    volatile double py = ly * (double)lv->h;
    x = px - 0.5;
    y = py - 0.5;
  }
  memset(g, 0, sizeof(*g));
  g->in = lv->ok && x >= -1.0 && x < (double)lv->w && y >= -1.0 && y < (double)lv->h;
  if (!g->in) return;
  const double xf = floor(x), yf = floor(y);
  g->dx = x - xf;
  g->dy = y - yf;
  const int64_t x0 = (int64_t)xf, y0 = (int64_t)yf;
  const int64_t xs[4] = {x0, x0 + 1, x0, x0 + 1};
  const int64_t ys[4] = {y0, y0, y0 + 1, y0 + 1};
  const double wx[4] = {1.0 - g->dx, g->dx, 1.0 - g->dx, g->dx};
  const double wy[4] = {1.0 - g->dy, 1.0 - g->dy, g->dy, g->dy};
  for (int c = 0; c < 4; ++c) {
    g->mask[c] = xs[c] >= 0 && xs[c] < lv->w && ys[c] >= 0 && ys[c] < lv->h;
    g->pos[c] = g->mask[c] ? lv->start + ys[c] * lv->w + xs[c] : 0;
    g->w[c] = g->mask[c] ? wx[c] * wy[c] : 0.0;
  }
}

static int read_levels(const int64_t* shapes, const int64_t* starts, int64_t L, int64_t S,
                       level_t* levels) {
  for (int64_t l = 0; l < L; ++l) {
    const int64_t h = shapes[2 * l], w = shapes[2 * l + 1], st = starts[l];
    levels[l].h = h;
    levels[l].w = w;
    levels[l].start = st;
    levels[l].ok = h > 0 && w > 0 && st >= 0 && st + h * w <= S;
  }
  return 0;
}

/* Normalized weights of one (b, q, h): attn as given, or its softmax. */
static void unit_weights(const double* attn, int64_t LP, int softmax, double* p) {
  if (!softmax) {
    for (int64_t s = 0; s < LP; ++s) p[s] = attn[s];
    return;
  }
  double mx = -INFINITY, sum = 0.0;
  for (int64_t s = 0; s < LP; ++s) mx = attn[s] > mx ? attn[s] : mx;
  for (int64_t s = 0; s < LP; ++s) sum += exp(attn[s] - mx);
  for (int64_t s = 0; s < LP; ++s) p[s] = exp(attn[s] - mx) / sum;
}

int msda_oracle_forward(const double* value, const int64_t* shapes, const int64_t* starts,
                        const double* loc, const double* attn, double* out, int64_t B, int64_t S,
                        int64_t H, int64_t D, int64_t Q, int64_t L, int64_t P, int softmax,
                        int pixel_f32) {
  const int64_t LP = L * P;
  level_t* levels = (level_t*)malloc(sizeof(level_t) * (size_t)(L > 0 ? L : 1));
  double* p = (double*)malloc(sizeof(double) * (size_t)(LP > 0 ? LP : 1));
  if (!levels || !p) return 1;
  read_levels(shapes, starts, L, S, levels);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t q = 0; q < Q; ++q)
      for (int64_t h = 0; h < H; ++h) {
        const int64_t unit = (b * Q + q) * H + h;
        double* o = out + unit * D;
        for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
        unit_weights(attn + unit * LP, LP, softmax, p);
        for (int64_t s = 0; s < LP; ++s) {
          geom_t g;
          geometry(loc[(unit * LP + s) * 2], loc[(unit * LP + s) * 2 + 1], &levels[s / P],
                   pixel_f32, &g);
          if (!g.in) continue;
          for (int c = 0; c < 4; ++c) {
            if (!g.mask[c]) continue;
            const double* v = value + ((b * S + g.pos[c]) * H + h) * D;
            const double wa = g.w[c] * p[s];
            for (int64_t d = 0; d < D; ++d) o[d] += wa * v[d];
          }
        }
      }
  free(levels);
  free(p);
  return 0;
}

int msda_oracle_backward(const double* value, const int64_t* shapes, const int64_t* starts,
                         const double* loc, const double* attn, const double* grad_out,
                         double* grad_value, double* grad_loc, double* grad_attn, int64_t B,
                         int64_t S, int64_t H, int64_t D, int64_t Q, int64_t L, int64_t P,
                         int softmax, int pixel_f32) {
  const int64_t LP = L * P;
  level_t* levels = (level_t*)malloc(sizeof(level_t) * (size_t)(L > 0 ? L : 1));
  double* p = (double*)malloc(sizeof(double) * (size_t)(LP > 0 ? LP : 1));
  double* gp = (double*)malloc(sizeof(double) * (size_t)(LP > 0 ? LP : 1));
  if (!levels || !p || !gp) return 1;
  read_levels(shapes, starts, L, S, levels);
  memset(grad_value, 0, sizeof(double) * (size_t)(B * S * H * D));
  for (int64_t b = 0; b < B; ++b)
    for (int64_t q = 0; q < Q; ++q)
      for (int64_t h = 0; h < H; ++h) {
        const int64_t unit = (b * Q + q) * H + h;
        const double* g_out = grad_out + unit * D;
        unit_weights(attn + unit * LP, LP, softmax, p);
        for (int64_t s = 0; s < LP; ++s) {
          const level_t* lv = &levels[s / P];
          double* gl = grad_loc + (unit * LP + s) * 2;
          geom_t g;
          geometry(loc[(unit * LP + s) * 2], loc[(unit * LP + s) * 2 + 1], lv, pixel_f32, &g);
          gl[0] = gl[1] = 0.0;
          gp[s] = 0.0;
          if (!g.in) continue;
          double G[4] = {0.0, 0.0, 0.0, 0.0};
          for (int c = 0; c < 4; ++c) {
            if (!g.mask[c]) continue;
            const int64_t base = ((b * S + g.pos[c]) * H + h) * D;
            const double wa = g.w[c] * p[s];
            for (int64_t d = 0; d < D; ++d) {
              G[c] += g_out[d] * value[base + d];
              grad_value[base + d] += wa * g_out[d];
            }
          }
          gp[s] = g.w[0] * G[0] + g.w[1] * G[1] + g.w[2] * G[2] + g.w[3] * G[3];
          gl[0] = p[s] * (double)lv->w * ((1.0 - g.dy) * (G[1] - G[0]) + g.dy * (G[3] - G[2]));
          gl[1] = p[s] * (double)lv->h * ((1.0 - g.dx) * (G[2] - G[0]) + g.dx * (G[3] - G[1]));
        }
        double* ga = grad_attn + unit * LP;
        if (softmax) {
          double dot = 0.0;
          for (int64_t s = 0; s < LP; ++s) dot += p[s] * gp[s];
          for (int64_t s = 0; s < LP; ++s) ga[s] = p[s] * (gp[s] - dot);
        } else {
          for (int64_t s = 0; s < LP; ++s) ga[s] = gp[s];
        }
      }
  free(levels);
  free(p);
  free(gp);
  return 0;
}
