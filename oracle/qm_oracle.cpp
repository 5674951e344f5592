// qm38 CPU ORACLE — test infrastructure only.
//
// A scalar C++ restatement of the reference's per-token compute path
// (/root/reference, Fuxx-1/qwen38-metal), used ONLY by tests/, by
// __graft_entry__.smoke() and by bench.py's cpu_baseline leg, as the checker
// and as the reported CPU baseline.  The product (qwen38-metal_amd/) never
// links or calls it.
//
// Each function cites the reference code whose semantics it restates.  The
// reference is Rust + Metal and cannot be built here (no cargo, no xcrun),
// so there is no oracle/_ref build; the restatement is pinned by the
// reference's own test vectors and by closed forms (tests/test_oracle.py).
//
// Build: make -C oracle  (gcc, -O2 -fopenmp -ffp-contract=off, no fast-math:
// the Q8 quantiser relies on IEEE division and round-half-away-from-zero).
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

extern "C" {

// qwen38.metal:18-20 / metal_runtime.rs:12134-12136
float qo_bf16_to_f32(uint16_t v) {
  uint32_t bits = (uint32_t)v << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// qwen38.metal:22-26 / metal_runtime.rs:12128-12132 (RNE via +0x7fff+lsb)
uint16_t qo_f32_to_bf16(float f) {
  uint32_t bits;
  memcpy(&bits, &f, 4);
  return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

static inline uint32_t nibble(const uint32_t* row_words, uint32_t i) {
  return (row_words[i >> 3] >> (4 * (i & 7))) & 0xFu;
}

// MLX affine-Q4 projection, the math of qwen38_q4_affine_matvec /
// _matvec_simd (qwen38.metal:213-246, 815-867):
//   y[m][n] = sum_g ( s[n][g] * sum_{i in g} q[n][i] x[m][i]
//                   + b[n][g] * sum_{i in g} x[m][i] )
// Word w of a row holds q[8w..8w+7], value j at bits 4j..4j+3
// (qwen38.metal:28-43, pack_q4 metal_runtime.rs:11962-11975).
// x is bf16 [M][K]; y fp32 [M][N]; accumulation in double.
void qo_q4_project(const uint16_t* x, uint32_t M, uint32_t K, const uint32_t* w, const uint16_t* s,
                   const uint16_t* b, uint32_t N, float* y, int threads) {
  const uint32_t G = K / 64, WPR = K / 8;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) if (threads != 1)
#endif
  for (int64_t n = 0; n < (int64_t)N; ++n) {
    const uint32_t* row = w + (size_t)n * WPR;
    for (uint32_t m = 0; m < M; ++m) {
      const uint16_t* xr = x + (size_t)m * K;
      double total = 0.0;
      for (uint32_t g = 0; g < G; ++g) {
        double dot = 0.0, sum = 0.0;
        for (uint32_t i = g * 64; i < g * 64 + 64; ++i) {
          const double xv = qo_bf16_to_f32(xr[i]);
          dot += (double)nibble(row, i) * xv;
          sum += xv;
        }
        total += (double)qo_bf16_to_f32(s[(size_t)n * G + g]) * dot + (double)qo_bf16_to_f32(b[(size_t)n * G + g]) * sum;
      }
      y[(size_t)m * N + n] = (float)total;
    }
  }
}

// Same math in fp32 with the reference kernel's per-group accumulation order
// (qwen38_q4_affine_matvec_simd, qwen38.metal:224-240), multithreaded over
// output rows: the CPU baseline of the decode projection.
void qo_q4_project_f32(const uint16_t* x, uint32_t M, uint32_t K, const uint32_t* w, const uint16_t* s,
                       const uint16_t* b, uint32_t N, float* y, int threads) {
  const uint32_t G = K / 64, WPR = K / 8;
  std::vector<float> xf((size_t)M * K);
  for (size_t i = 0; i < xf.size(); ++i) xf[i] = qo_bf16_to_f32(x[i]);
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) if (threads != 1)
#endif
  for (int64_t n = 0; n < (int64_t)N; ++n) {
    const uint32_t* row = w + (size_t)n * WPR;
    for (uint32_t m = 0; m < M; ++m) {
      const float* xr = xf.data() + (size_t)m * K;
      float total = 0.f;
      for (uint32_t g = 0; g < G; ++g) {
        float dot = 0.f, sum = 0.f;
        for (uint32_t wd = 0; wd < 8; ++wd) {
          const uint32_t p = row[g * 8 + wd];
          const float* xv = xr + g * 64 + wd * 8;
          for (int j = 0; j < 8; ++j) {
            dot += (float)((p >> (4 * j)) & 0xFu) * xv[j];
            sum += xv[j];
          }
        }
        total += dot * qo_bf16_to_f32(s[(size_t)n * G + g]) + sum * qo_bf16_to_f32(b[(size_t)n * G + g]);
      }
      y[(size_t)m * N + n] = total;
    }
  }
}

// silu(g) * u with silu(v) = v * (1 / (1 + exp(-v)))
// (qwen38_swiglu_rows, qwen38.metal:4090-4096, 4188-4199).
void qo_swiglu(const float* g, const float* u, size_t n, float* h) {
  for (size_t i = 0; i < n; ++i) {
    const float sg = 1.0f / (1.0f + expf(-g[i]));
    h[i] = g[i] * sg * u[i];
  }
}

// Q8 K/V quantisation of one (token, kv_head) row of `d` values
// (qwen38_q8_kv_append, qwen38.metal:5031-5080):
//   scale = max(absmax / 127, FLT_MIN)
//   q_i   = char(round(clamp(x_i / scale, -127, 127)))   (round half away)
void qo_q8_quantize(const float* x, uint32_t d, int8_t* q, float* scale) {
  float a = 0.f;
  for (uint32_t i = 0; i < d; ++i) a = fmaxf(a, fabsf(x[i]));
  const float s = fmaxf(a / 127.0f, FLT_MIN);
  *scale = s;
  for (uint32_t i = 0; i < d; ++i) {
    const float v = fminf(fmaxf(x[i] / s, -127.0f), 127.0f);
    q[i] = (int8_t)roundf(v);
  }
}

// Row-wise qo_q8_quantize of n rows of d elements (scales [n]).
void qo_q8_quantize_rows(const float* x, uint64_t n, uint32_t d, int8_t* q, float* scale) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t r = 0; r < (int64_t)n; ++r) qo_q8_quantize(x + (size_t)r * d, d, q + (size_t)r * d, scale + r);
}

// GQA attention of `rows` query rows over a token-major Q8 cache
// (Q8KvState layout, metal_runtime.rs:578-593):
//   keys/values int8 [T][KVH][d], key/value scales fp32 [T][KVH].
// Row r sees tokens [0, visible_r) with visible_r = min(start + r + 1, total)
// (qwen38_gqa_q8_prefill_attention, qwen38.metal:5146-5238); decode is the
// case rows = 1, start = total - 1 (qwen38_gqa_q8_scores/values,
// qwen38.metal:5240-5323).  Head h uses KV head h*KVH/H.
//   s_t = (sum_d q_d K_td ks_t) / sqrt(d);  p = softmax(s);
//   o_d = sum_t p_t V_td vs_t * sigmoid(gate_d)   (gate may be NULL: no gate)
// q, gate: fp32 [rows][H][d]; o fp32 [rows][H][d].  Double accumulation.
void qo_attention(const float* q, const float* gate, const int8_t* keys, const float* kscale,
                  const int8_t* values, const float* vscale, uint32_t rows, uint32_t H, uint32_t KVH,
                  uint32_t d, uint32_t start, uint32_t total, float* o, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic) if (threads != 1)
#endif
  for (int64_t rh = 0; rh < (int64_t)rows * H; ++rh) {
    const uint32_t r = (uint32_t)(rh / H), h = (uint32_t)(rh % H);
    const uint32_t kvh = h * KVH / H;
    uint32_t visible = start + r + 1;
    if (visible > total) visible = total;
    const float* qr = q + ((size_t)r * H + h) * d;
    std::vector<double> sc(visible);
    double mx = -INFINITY;
    for (uint32_t t = 0; t < visible; ++t) {
      const int8_t* kr = keys + ((size_t)t * KVH + kvh) * d;
      double dot = 0.0;
      for (uint32_t i = 0; i < d; ++i) dot += (double)qr[i] * (double)kr[i];
      dot = dot * (double)kscale[(size_t)t * KVH + kvh] / sqrt((double)d);
      sc[t] = dot;
      if (dot > mx) mx = dot;
    }
    double den = 0.0;
    for (uint32_t t = 0; t < visible; ++t) {
      sc[t] = exp(sc[t] - mx);
      den += sc[t];
    }
    float* orow = o + ((size_t)r * H + h) * d;
    // Token-outer so each V row is read once; every acc[i] still sums its
    // terms sc_t * v_ti * vs_t in token order.
    std::vector<double> accv(d, 0.0);
    for (uint32_t t = 0; t < visible; ++t) {
      const int8_t* vr = values + ((size_t)t * KVH + kvh) * d;
      const double w = sc[t], vs = (double)vscale[(size_t)t * KVH + kvh];
      for (uint32_t i = 0; i < d; ++i) accv[i] += w * (double)vr[i] * vs;
    }
    for (uint32_t i = 0; i < d; ++i) {
      double acc = accv[i];
      acc /= den;
      if (gate) acc *= 1.0 / (1.0 + exp(-(double)gate[((size_t)r * H + h) * d + i]));
      orow[i] = (float)acc;
    }
  }
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Gated DeltaNet, one token (deltanet_step, metal_runtime.rs:7459-7636), in
// the reference kernels' operation order:
//   conv      qwen38_deltanet_conv        qwen38.metal:4376-4402
//   prepare   qwen38_deltanet_prepare     qwen38.metal:4405-4446
//   recurrence qwen38_deltanet_recurrence qwen38.metal:4449-4495
//   gate norm qwen38_deltanet_gate_norm   qwen38.metal:4497-4527
// channels = 2*KH*dk + VH*dv; qkv [channels] = [q (KH*dk) | k (KH*dk) | v]
// conv_w [channels][ks]; hist [channels][ks-1]; S [VH][dv][dk].
// T = float mirrors the reference in fp32; T = double is a higher-precision
// twin used to bound the fp32 oracle's own rounding.
template <typename T>
static T t_sigmoid(T v) { return T(1) / (T(1) + exp(-v)); }
template <typename T>
static T t_softplus(T v) {
  if (v > T(20)) return v;
  if (v < T(-20)) return exp(v);
  return log(T(1) + exp(v));
}

template <typename T>
static void dn_step(uint32_t KH, uint32_t VH, uint32_t dk, uint32_t dv, uint32_t ks, const float* conv_w,
                    const float* a_log, const float* dt_bias, const float* norm, const float* qkv, const float* z,
                    const float* b, const float* a, float eps, T* hist, T* S, float* out) {
  const uint32_t key_el = KH * dk, channels = 2 * key_el + VH * dv, hw = ks - 1;
  std::vector<T> c(channels);
  for (uint32_t ch = 0; ch < channels; ++ch) {
    T sum = (T)conv_w[(size_t)ch * ks + hw] * (T)qkv[ch];
    for (uint32_t tap = 0; tap < hw; ++tap) sum += (T)conv_w[(size_t)ch * ks + tap] * hist[(size_t)ch * hw + tap];
    c[ch] = sum * t_sigmoid<T>(sum);
    if (hw > 0) {
      for (uint32_t tap = 0; tap + 1 < hw; ++tap) hist[(size_t)ch * hw + tap] = hist[(size_t)ch * hw + tap + 1];
      hist[(size_t)ch * hw + hw - 1] = (T)qkv[ch];
    }
  }
  const T inv = T(1) / sqrt((T)dk);
  for (uint32_t h = 0; h < KH; ++h) {
    T qs = 0, kss = 0;
    for (uint32_t i = 0; i < dk; ++i) {
      qs += c[h * dk + i] * c[h * dk + i];
      kss += c[key_el + h * dk + i] * c[key_el + h * dk + i];
    }
    const T qscale = T(1) / sqrt(qs / (T)dk + (T)eps), kscale = T(1) / sqrt(kss / (T)dk + (T)eps);
    for (uint32_t i = 0; i < dk; ++i) {
      c[h * dk + i] = c[h * dk + i] * qscale * inv * inv;
      c[key_el + h * dk + i] = c[key_el + h * dk + i] * kscale * inv;
    }
  }
  const uint32_t rep = VH / KH;
  // Value heads are independent: they run on OpenMP threads (each head's
  // arithmetic is unchanged).
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (VH > 1)
#endif
  for (uint32_t vh = 0; vh < VH; ++vh) {
    std::vector<T> o(dv);
    const uint32_t kh = vh / rep;
    const T* qv = &c[kh * dk];
    const T* kv = &c[key_el + kh * dk];
    const T decay = exp(-exp((T)a_log[vh]) * t_softplus<T>((T)a[vh] + (T)dt_bias[vh]));
    const T beta = t_sigmoid<T>((T)b[vh]);
    for (uint32_t i = 0; i < dv; ++i) {
      T* row = S + ((size_t)vh * dv + i) * dk;
      T mem = 0;
      for (uint32_t j = 0; j < dk; ++j) {
        row[j] = row[j] * decay;
        mem += row[j] * kv[j];
      }
      const T delta = (c[2 * key_el + vh * dv + i] - mem) * beta;
      T acc = 0;
      for (uint32_t j = 0; j < dk; ++j) {
        row[j] = row[j] + kv[j] * delta;
        acc += row[j] * qv[j];
      }
      o[i] = acc;
    }
    T ss = 0;
    for (uint32_t i = 0; i < dv; ++i) ss += o[i] * o[i];
    const T scale = T(1) / sqrt(ss / (T)dv + (T)eps);
    for (uint32_t i = 0; i < dv; ++i) {
      const T zz = (T)z[vh * dv + i];
      out[vh * dv + i] = (float)(o[i] * scale * (T)norm[i] * (zz * t_sigmoid<T>(zz)));
    }
  }
}

extern "C" {

// M tokens in sequence (qwen38_deltanet_prefill, qwen38.metal:4530-4758,
// equals M deltanet_step calls: metal_runtime.rs:11202-11260).  Activations
// have a leading [M] dimension.  hist/S are updated in place (fp32).
void qo_dn_prefill_f32(uint32_t KH, uint32_t VH, uint32_t dk, uint32_t dv, uint32_t ks, const float* conv_w,
                       const float* a_log, const float* dt_bias, const float* norm, const float* qkv,
                       const float* z, const float* b, const float* a, uint32_t M, float eps, float* hist,
                       float* S, float* out) {
  const size_t channels = 2 * (size_t)KH * dk + (size_t)VH * dv;
  for (uint32_t t = 0; t < M; ++t)
    dn_step<float>(KH, VH, dk, dv, ks, conv_w, a_log, dt_bias, norm, qkv + t * channels, z + (size_t)t * VH * dv,
                   b + (size_t)t * VH, a + (size_t)t * VH, eps, hist, S, out + (size_t)t * VH * dv);
}

// Double-precision twin; hist/S are double here.
void qo_dn_prefill_f64(uint32_t KH, uint32_t VH, uint32_t dk, uint32_t dv, uint32_t ks, const float* conv_w,
                       const float* a_log, const float* dt_bias, const float* norm, const float* qkv,
                       const float* z, const float* b, const float* a, uint32_t M, float eps, double* hist,
                       double* S, float* out) {
  const size_t channels = 2 * (size_t)KH * dk + (size_t)VH * dv;
  for (uint32_t t = 0; t < M; ++t)
    dn_step<double>(KH, VH, dk, dv, ks, conv_w, a_log, dt_bias, norm, qkv + t * channels, z + (size_t)t * VH * dv,
                    b + (size_t)t * VH, a + (size_t)t * VH, eps, hist, S, out + (size_t)t * VH * dv);
}

// Full-attention q/k preparation for M rows: per-head RMSNorm with a learned
// weight, partial (M-)RoPE on the first rotary_dim dims, query/gate split.
//   q_with_gate [M][H][2 hd]  (query | gate per head; split_query_and_gate,
//                              native.rs:4917-4942)
//   k_in        [M][KVH][hd]
//   positions   [3][M] (axis-major) or NULL: every axis = base + row
// RMSNorm follows rms_norm_slice (native.rs:5153-5161): mean of squares
// summed in order, scale = 1/sqrt(mean + eps), out = x * scale * w.  RoPE
// follows apply_mrope (native.rs:5163-5180) with the interleaved axis choice
// of MropePosition::axis_for_frequency (native.rs:136-148) and the GPU
// kernels qwen38_gqa_prepare_query(_rows) / _key(_rows) (qwen38.metal:
// 4761-5029).  One deviation: the reference forms the angle pos /
// theta^(2i/rd) in fp32, where one ulp of powf moves the angle by ~1e-2 rad
// at positions near 128K; here (and in the HIP kernel) frequency, angle and
// sin/cos are evaluated in fp64 and rounded to fp32.
static void prep_head(const float* x, const float* w, uint32_t hd, uint32_t rd, double theta, uint32_t s1, uint32_t s2,
                      uint32_t has_sections, const uint32_t pos[3], float eps, float* out) {
  float sum = 0.0f;
  for (uint32_t i = 0; i < hd; ++i) sum += x[i] * x[i];
  const float mean = sum / (float)hd;
  const float scale = 1.0f / sqrtf(mean + eps);
  for (uint32_t i = 0; i < hd; ++i) out[i] = x[i] * scale * w[i];
  const uint32_t half = rd / 2;
  for (uint32_t i = 0; i < half; ++i) {
    uint32_t p = pos[0];
    if (has_sections) {
      if (i % 3 == 1 && i / 3 < s1) p = pos[1];
      if (i % 3 == 2 && i / 3 < s2) p = pos[2];
    }
    const double angle = (double)p / pow(theta, (double)(2 * i) / (double)rd);
    const float sn = (float)sin(angle), cs = (float)cos(angle);
    const float left = out[i], right = out[i + half];
    out[i] = left * cs - right * sn;
    out[i + half] = right * cs + left * sn;
  }
}

void qo_attn_prepare(const float* q_with_gate, const float* k_in, const float* q_norm, const float* k_norm,
                     uint32_t M, uint32_t H, uint32_t KVH, uint32_t hd, uint32_t rd, double theta, uint32_t s1,
                     uint32_t s2, uint32_t has_sections, const uint32_t* positions, uint32_t base, float eps,
                     float* q_out, float* gate_out, float* k_out) {
  for (uint32_t r = 0; r < M; ++r) {
    uint32_t pos[3];
    for (int a = 0; a < 3; ++a) pos[a] = positions ? positions[(size_t)a * M + r] : base + r;
    for (uint32_t h = 0; h < H; ++h) {
      const float* src = q_with_gate + ((size_t)r * H + h) * 2 * hd;
      prep_head(src, q_norm, hd, rd, theta, s1, s2, has_sections, pos, eps, q_out + ((size_t)r * H + h) * hd);
      memcpy(gate_out + ((size_t)r * H + h) * hd, src + hd, hd * sizeof(float));
    }
    for (uint32_t h = 0; h < KVH; ++h)
      prep_head(k_in + ((size_t)r * KVH + h) * hd, k_norm, hd, rd, theta, s1, s2, has_sections, pos, eps,
                k_out + ((size_t)r * KVH + h) * hd);
  }
}

// Residual add + RMSNorm of M rows (qwen38_add_in_place followed by
// qwen38_rms_norm / qwen38_rms_norm_rows, shaders/qwen38.metal:4253-4333):
// hidden += delta (when delta != NULL), then
// out = hidden * (1 / sqrt(mean(hidden^2) + eps)) * w, the weights used as
// given.  hidden is updated in fp32 (the reference's type); the norm is
// evaluated in fp64 and returned unrounded.
void qo_residual_rmsnorm(float* hidden, const float* delta, const float* w, uint32_t M, uint32_t n, float eps,
                         double* out) {
  for (uint32_t r = 0; r < M; ++r) {
    float* h = hidden + (size_t)r * n;
    if (delta)
      for (uint32_t i = 0; i < n; ++i) h[i] = h[i] + delta[(size_t)r * n + i];
    double ss = 0.0;
    for (uint32_t i = 0; i < n; ++i) ss += (double)h[i] * h[i];
    const double scale = 1.0 / std::sqrt(ss / n + (double)eps);
    for (uint32_t i = 0; i < n; ++i) out[(size_t)r * n + i] = (double)h[i] * scale * (double)w[i];
  }
}

int qo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

}  // extern "C"
