// TEST INFRASTRUCTURE ONLY. The CPU oracle: a float32 restatement of relay's CPU
// backend (engine/src/cpu_backend.cpp) and of the host-side conversions its CUDA
// backend relies on. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
// leg may load it, and only as the checker or the timed CPU baseline; the product
// (relay_amd) never calls into it.
//
// Bitwise contract: built with -O3 -ffp-contract=off and no -march flag (see Makefile),
// forward() gives the same bits as the reference's CpuBackend built the same way, because
// every output element is produced by the same sequence of float operations:
//   - dot: 8 independent partial sums, combined ((0+1)+(2+3))+((4+5)+(6+7)) + tail
//     (cpu_backend.cpp:20-28);
//   - matmul: y[t,n] = dot(x[t], W[n]) (+ y[t,n]) (cpu_backend.cpp:31-45);
//   - rmsnorm: double sum of squares, float inverse root, w * (x * inv) (cpu_backend.cpp:47-52);
//   - RoPE with cosf/sinf of pos * inv_freq[i], rotate_half pairs (cpu_backend.cpp:223-235);
//   - attention: scores dot * scale, expf(s - max), p = e / sum, out += p * v in key
//     order (cpu_backend.cpp:152-180);
//   - SiLU g / (1 + expf(-g)) * u (cpu_backend.cpp:188-194).
// Pinned by tests/test_oracle.py: bitwise against the reference CPU backend compiled from
// /root/reference (oracle/_ref, when present) and against the committed goldens made
// from it, and against the Hugging Face logits in the reference's fixtures.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;

// Same layout as rh_model_config in include/relay_hip.h (the tests share one ctypes struct).
struct OracleConfig {
  int hidden, intermediate, layers, heads, kv_heads, head_dim, vocab, tie_embeddings, qkv_bias;
  int rope_scaling_llama3;
  double rms_eps, rope_theta, rope_factor, rope_low_freq_factor, rope_high_freq_factor, rope_original_max_position;
};

inline float dot8(const float* a, const float* b, int n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int i = 0;
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; ++l) acc[l] += a[i + l] * b[i + l];
  float tail = 0;
  for (; i < n; ++i) tail += a[i] * b[i];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7])) + tail;
}

void matmul(const float* x, const float* W, float* y, int T, int K, int N, bool accumulate) {
  // Rows of W in groups of 16 per OpenMP iteration, as cpu_backend.cpp:31-45; the
  // grouping only distributes work, each element's arithmetic is dot8.
#pragma omp parallel for schedule(static)
  for (int n0 = 0; n0 < N; n0 += 16) {
    const int n1 = std::min(N, n0 + 16);
    for (int t = 0; t < T; ++t) {
      const float* xt = x + static_cast<std::int64_t>(t) * K;
      float* yt = y + static_cast<std::int64_t>(t) * N;
      for (int n = n0; n < n1; ++n) {
        const float v = dot8(xt, W + static_cast<std::int64_t>(n) * K, K);
        yt[n] = accumulate ? yt[n] + v : v;
      }
    }
  }
}

void rmsnorm(const float* x, const float* w, float* out, int n, float eps) {
  double ss = 0;
  for (int i = 0; i < n; ++i) ss += static_cast<double>(x[i]) * x[i];
  const float inv = 1.0f / std::sqrt(static_cast<float>(ss / n) + eps);
  for (int i = 0; i < n; ++i) out[i] = w[i] * (x[i] * inv);
}

// config.cpp:79-109: 1 / theta^(2i/d) in float, then Llama 3 band scaling.
std::vector<float> rope_inv_freq(const OracleConfig& c) {
  const int half = c.head_dim / 2;
  std::vector<float> inv(half);
  for (int i = 0; i < half; ++i) {
    const float e = static_cast<float>(2 * i) / static_cast<float>(c.head_dim);
    inv[i] = 1.0f / std::pow(static_cast<float>(c.rope_theta), e);
  }
  if (c.rope_scaling_llama3) {
    const double low_wavelen = c.rope_original_max_position / c.rope_low_freq_factor;
    const double high_wavelen = c.rope_original_max_position / c.rope_high_freq_factor;
    for (int i = 0; i < half; ++i) {
      const float f = inv[i];
      const float wavelen = 2.0f * static_cast<float>(3.14159265358979323846) / f;
      float r = wavelen > low_wavelen ? f / static_cast<float>(c.rope_factor) : f;
      if (!(wavelen < high_wavelen) && !(wavelen > low_wavelen)) {
        const float smooth = static_cast<float>((c.rope_original_max_position / wavelen - c.rope_low_freq_factor) /
                                                (c.rope_high_freq_factor - c.rope_low_freq_factor));
        r = (1 - smooth) * f / static_cast<float>(c.rope_factor) + smooth * f;
      }
      inv[i] = r;
    }
  }
  return inv;
}

// IEEE binary32 -> binary16, round to nearest, ties to even; NaN stays a quiet NaN,
// overflow goes to infinity (safetensors.cpp:65-89 computes the same function).
std::uint16_t to_f16(float f) {
  std::uint32_t x;
  std::memcpy(&x, &f, 4);
  const std::uint32_t sign = (x >> 16) & 0x8000u;
  const std::uint32_t exp = (x >> 23) & 0xFFu;
  std::uint32_t mant = x & 0x7FFFFFu;
  if (exp == 0xFFu) return static_cast<std::uint16_t>(sign | 0x7C00u | (mant ? 0x200u : 0u));
  const int e = static_cast<int>(exp) - 112;  // rebias 127 -> 15
  if (e >= 31) return static_cast<std::uint16_t>(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return static_cast<std::uint16_t>(sign);
    mant |= 0x800000u;
    const int shift = 14 - e;
    std::uint32_t h = mant >> shift;
    const std::uint32_t rem = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (h & 1u))) ++h;
    return static_cast<std::uint16_t>(sign | h);
  }
  std::uint32_t h = sign | (static_cast<std::uint32_t>(e) << 10) | (mant >> 13);
  const std::uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry into the exponent is correct rounding
  return static_cast<std::uint16_t>(h);
}

float from_f16(std::uint16_t h) {
  const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
  std::uint32_t exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      exp = 113;
      while (!(mant & 0x400u)) {
        mant <<= 1;
        --exp;
      }
      bits = sign | (exp << 23) | ((mant & 0x3FFu) << 13);
    }
  } else if (exp == 0x1Fu) {
    bits = sign | 0x7F800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

struct Model {
  OracleConfig c;
  // Borrowed fp32 weights (the caller keeps them alive), relay's fused layout.
  const float* embed;
  const float* final_norm;
  const float* lm_head;
  std::vector<const float*> attn_norm, wqkv, bqkv, wo, mlp_norm, w_gate_up, w_down;
  int num_blocks, block_size;
  std::vector<float> k, v;  // [layer][block][kv_head][slot][D]
  std::vector<float> inv_freq;

  std::int64_t block_elems() const { return static_cast<std::int64_t>(c.kv_heads) * block_size * c.head_dim; }
  std::int64_t layer_elems() const { return block_elems() * num_blocks; }
  std::int64_t offset(int block, int kvh, int slot) const {
    return (static_cast<std::int64_t>(block) * c.kv_heads + kvh) * block_size * c.head_dim +
           static_cast<std::int64_t>(slot) * c.head_dim;
  }

  void rope(float* x, int nheads, int p) const {
    const int D = c.head_dim, half = D / 2;
    for (int i = 0; i < half; ++i) {
      const float angle = static_cast<float>(p) * inv_freq[i];
      const float cs = std::cos(angle), sn = std::sin(angle);
      for (int h = 0; h < nheads; ++h) {
        float* r = x + h * D;
        const float a = r[i], b = r[i + half];
        r[i] = a * cs - b * sn;
        r[i + half] = b * cs + a * sn;
      }
    }
  }
};

struct Batch {
  std::vector<int> n_tokens, start_pos, table_len, want;
  std::vector<std::vector<int>> tok, table;
  bool all_logits;
};

// CpuBackend::forward restated (cpu_backend.cpp:90-218). Returns logits rows.
std::vector<float> forward(Model& m, const Batch& b) {
  const OracleConfig& c = m.c;
  const int H = c.hidden, Q = c.heads * c.head_dim, KV = c.kv_heads * c.head_dim, I = c.intermediate,
            D = c.head_dim;
  const int QKV = Q + 2 * KV, S = static_cast<int>(b.tok.size());
  std::vector<int> tok, pos, seq_of;
  for (int s = 0; s < S; ++s) {
    const int need = (b.start_pos[s] + b.n_tokens[s] + m.block_size - 1) / m.block_size;
    if (b.table_len[s] < need) throw std::invalid_argument("block table too short");
    for (int blk : b.table[s])
      if (blk < 0 || blk >= m.num_blocks) throw std::invalid_argument("block id outside the cache");
    for (int i = 0; i < b.n_tokens[s]; ++i) {
      tok.push_back(b.tok[s][i]);
      pos.push_back(b.start_pos[s] + i);
      seq_of.push_back(s);
    }
  }
  const int T = static_cast<int>(tok.size());
  if (T == 0) return {};
  std::vector<float> x(static_cast<std::size_t>(T) * H), xn(x.size());
  std::vector<float> qkv(static_cast<std::size_t>(T) * QKV), attn(static_cast<std::size_t>(T) * Q);
  std::vector<float> gu(static_cast<std::size_t>(T) * 2 * I), act(static_cast<std::size_t>(T) * I);
  for (int t = 0; t < T; ++t) {
    if (tok[t] < 0 || tok[t] >= c.vocab) throw std::out_of_range("token id out of range");
    std::memcpy(&x[static_cast<std::size_t>(t) * H], m.embed + static_cast<std::size_t>(tok[t]) * H, H * 4);
  }
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));
  const int group = c.heads / c.kv_heads;
  const float eps = static_cast<float>(c.rms_eps);

  for (int l = 0; l < c.layers; ++l) {
    float* Kc = m.k.data() + l * m.layer_elems();
    float* Vc = m.v.data() + l * m.layer_elems();
#pragma omp parallel for
    for (int t = 0; t < T; ++t)
      rmsnorm(&x[static_cast<std::size_t>(t) * H], m.attn_norm[l], &xn[static_cast<std::size_t>(t) * H], H, eps);
    matmul(xn.data(), m.wqkv[l], qkv.data(), T, H, QKV, false);
#pragma omp parallel for
    for (int t = 0; t < T; ++t) {
      float* row = &qkv[static_cast<std::size_t>(t) * QKV];
      if (m.bqkv[l])
        for (int i = 0; i < QKV; ++i) row[i] += m.bqkv[l][i];
      m.rope(row, c.heads, pos[t]);
      m.rope(row + Q, c.kv_heads, pos[t]);
      const int s = seq_of[t];
      const int blk = b.table[s][pos[t] / m.block_size], slot = pos[t] % m.block_size;
      for (int h = 0; h < c.kv_heads; ++h) {
        const std::int64_t off = m.offset(blk, h, slot);
        std::memcpy(Kc + off, row + Q + h * D, D * 4);
        std::memcpy(Vc + off, row + Q + KV + h * D, D * 4);
      }
    }
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int t = 0; t < T; ++t) {
      for (int h = 0; h < c.heads; ++h) {
        const std::vector<int>& table = b.table[seq_of[t]];
        const float* q = &qkv[static_cast<std::size_t>(t) * QKV + h * D];
        const int kvh = h / group, n = pos[t] + 1;
        std::vector<float> score(n);
        float mx = -INFINITY;
        for (int j = 0; j < n; ++j) {
          score[j] = dot8(q, Kc + m.offset(table[j / m.block_size], kvh, j % m.block_size), D) * scale;
          mx = std::max(mx, score[j]);
        }
        float sum = 0;
        for (int j = 0; j < n; ++j) {
          score[j] = std::exp(score[j] - mx);
          sum += score[j];
        }
        float* out = &attn[static_cast<std::size_t>(t) * Q + h * D];
        std::fill(out, out + D, 0.0f);
        for (int j = 0; j < n; ++j) {
          const float* vr = Vc + m.offset(table[j / m.block_size], kvh, j % m.block_size);
          const float p = score[j] / sum;
          for (int d = 0; d < D; ++d) out[d] += p * vr[d];
        }
      }
    }
    matmul(attn.data(), m.wo[l], x.data(), T, Q, H, true);
#pragma omp parallel for
    for (int t = 0; t < T; ++t)
      rmsnorm(&x[static_cast<std::size_t>(t) * H], m.mlp_norm[l], &xn[static_cast<std::size_t>(t) * H], H, eps);
    matmul(xn.data(), m.w_gate_up[l], gu.data(), T, H, 2 * I, false);
#pragma omp parallel for
    for (int t = 0; t < T; ++t) {
      const float* g = &gu[static_cast<std::size_t>(t) * 2 * I];
      const float* u = g + I;
      float* a = &act[static_cast<std::size_t>(t) * I];
      for (int i = 0; i < I; ++i) a[i] = g[i] / (1.0f + std::exp(-g[i])) * u[i];
    }
    matmul(act.data(), m.w_down[l], x.data(), T, I, H, true);
  }
  std::vector<int> rows;
  int t0 = 0;
  for (int s = 0; s < S; ++s) {
    if (b.all_logits) {
      for (int i = 0; i < b.n_tokens[s]; ++i) rows.push_back(t0 + i);
    } else if (b.want[s]) {
      rows.push_back(t0 + b.n_tokens[s] - 1);
    }
    t0 += b.n_tokens[s];
  }
  const int R = static_cast<int>(rows.size());
  std::vector<float> xr(static_cast<std::size_t>(R) * H);
  for (int r = 0; r < R; ++r)
    rmsnorm(&x[static_cast<std::size_t>(rows[r]) * H], m.final_norm, &xr[static_cast<std::size_t>(r) * H], H, eps);
  std::vector<float> logits(static_cast<std::size_t>(R) * c.vocab);
  matmul(xr.data(), m.lm_head ? m.lm_head : m.embed, logits.data(), R, H, c.vocab, false);
  return logits;
}

template <class F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

}  // namespace

extern "C" {

const char* oracle_last_error(void) { return g_error.c_str(); }

void* oracle_model_new(const OracleConfig* cfg, const float* embed, const float* final_norm, const float* lm_head,
                       const float* const* attn_norm, const float* const* wqkv, const float* const* bqkv,
                       const float* const* wo, const float* const* mlp_norm, const float* const* w_gate_up,
                       const float* const* w_down, int num_blocks, int block_size) {
  Model* m = nullptr;
  int rc = guarded([&] {
    m = new Model();
    m->c = *cfg;
    m->embed = embed;
    m->final_norm = final_norm;
    m->lm_head = lm_head;
    const int L = cfg->layers;
    m->attn_norm.assign(attn_norm, attn_norm + L);
    m->wqkv.assign(wqkv, wqkv + L);
    m->bqkv = bqkv ? std::vector<const float*>(bqkv, bqkv + L) : std::vector<const float*>(L, nullptr);
    m->wo.assign(wo, wo + L);
    m->mlp_norm.assign(mlp_norm, mlp_norm + L);
    m->w_gate_up.assign(w_gate_up, w_gate_up + L);
    m->w_down.assign(w_down, w_down + L);
    m->num_blocks = num_blocks;
    m->block_size = block_size;
    m->k.assign(static_cast<std::size_t>(m->layer_elems() * L), 0.0f);
    m->v.assign(m->k.size(), 0.0f);
    m->inv_freq = rope_inv_freq(*cfg);
  });
  if (rc) {
    delete m;
    return nullptr;
  }
  return m;
}

void oracle_model_free(void* m) { delete static_cast<Model*>(m); }

// Flat batch (the same encoding as relay_hip_backend_forward). Returns rows, or -1.
int oracle_forward(void* mp, int n_seqs, const int* n_tokens, const int* tokens, const int* start_pos,
                   const int* table_len, const int* tables, const int* want_logits, int all_logits, float* logits,
                   size_t logits_cap) {
  Model& m = *static_cast<Model*>(mp);
  int rows = -1;
  int rc = guarded([&] {
    Batch b;
    b.all_logits = all_logits != 0;
    const int* tp = tokens;
    const int* bp = tables;
    for (int s = 0; s < n_seqs; ++s) {
      b.n_tokens.push_back(n_tokens[s]);
      b.start_pos.push_back(start_pos[s]);
      b.table_len.push_back(table_len[s]);
      b.want.push_back(want_logits ? want_logits[s] : 1);
      b.tok.emplace_back(tp, tp + n_tokens[s]);
      b.table.emplace_back(bp, bp + table_len[s]);
      tp += n_tokens[s];
      bp += table_len[s];
    }
    std::vector<float> lg = forward(m, b);
    if (lg.size() > logits_cap) throw std::invalid_argument("logits buffer too small");
    if (!lg.empty()) std::memcpy(logits, lg.data(), lg.size() * 4);
    rows = static_cast<int>(lg.size() / m.c.vocab);
  });
  return rc ? -1 : rows;
}

// The fp32 KV cache of one layer's block (read_kv_block, cpu_backend.cpp:73-77).
int oracle_read_kv_block(void* mp, int layer, int block, float* k_out, float* v_out) {
  Model& m = *static_cast<Model*>(mp);
  const std::int64_t off = layer * m.layer_elems() + block * m.block_elems();
  std::memcpy(k_out, m.k.data() + off, m.block_elems() * 4);
  std::memcpy(v_out, m.v.data() + off, m.block_elems() * 4);
  return 0;
}

int oracle_write_kv_block(void* mp, int layer, int block, const float* k_in, const float* v_in) {
  Model& m = *static_cast<Model*>(mp);
  const std::int64_t off = layer * m.layer_elems() + block * m.block_elems();
  std::memcpy(m.k.data() + off, k_in, m.block_elems() * 4);
  std::memcpy(m.v.data() + off, v_in, m.block_elems() * 4);
  return 0;
}

int oracle_rope_inv_freq(const OracleConfig* cfg, float* out) {
  std::vector<float> v = rope_inv_freq(*cfg);
  std::memcpy(out, v.data(), v.size() * 4);
  return 0;
}

void oracle_f32_to_f16(const float* in, std::uint16_t* out, size_t n) {
#pragma omp parallel for schedule(static) if (n > (1u << 16))
  for (size_t i = 0; i < n; ++i) out[i] = to_f16(in[i]);
}

void oracle_f16_to_f32(const std::uint16_t* in, float* out, size_t n) {
#pragma omp parallel for schedule(static) if (n > (1u << 16))
  for (size_t i = 0; i < n; ++i) out[i] = from_f16(in[i]);
}

// a[i] = the fp32 value of fp16(a[i]) (to_f16, then exact widening), in place.
void oracle_round_f16_inplace(float* a, size_t n) {
#pragma omp parallel for schedule(static) if (n > (1u << 16))
  for (size_t i = 0; i < n; ++i) a[i] = from_f16(to_f16(a[i]));
}

// The host int8 quantizer of cuda_backend.cu:282-304: per row, scale = max|w| / 127
// (1 when the row is zero), q = lrintf(w / scale).
void oracle_quantize_int8(const float* w, int N, int K, std::int8_t* q, float* scale) {
#pragma omp parallel for
  for (int n = 0; n < N; ++n) {
    const float* row = w + static_cast<std::size_t>(n) * K;
    float mx = 0.0f;
    for (int k = 0; k < K; ++k) mx = std::max(mx, std::fabs(row[k]));
    const float s = mx > 0.0f ? mx / 127.0f : 1.0f;
    scale[n] = s;
    for (int k = 0; k < K; ++k) q[static_cast<std::size_t>(n) * K + k] = static_cast<std::int8_t>(std::lrintf(row[k] / s));
  }
}

// Attention over a paged cache for a list of tokens, with the CPU backend's arithmetic
// (cpu_backend.cpp:152-180). The pools hold fp32 values (an fp16 cache widened exactly
// by the caller), laid out [block][kv_head][slot][D].
//   q: fp32 rows (row t at q + t * q_stride), heads * D values
//   out: fp32 rows (row i at out + i * heads * D) for the i-th listed token
void oracle_paged_attention(const float* q, long q_stride, const float* kpool, const float* vpool, const int* pos,
                            const int* seq, const int* table_off, const int* tables, const int* tokens, int n,
                            int heads, int kv_heads, int D, int block_size, float scale, float* out) {
  const int group = heads / kv_heads;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int i = 0; i < n; ++i) {
    for (int h = 0; h < heads; ++h) {
      const int t = tokens ? tokens[i] : i;
      const int* table = tables + table_off[seq[t]];
      const float* qr = q + static_cast<std::int64_t>(t) * q_stride + h * D;
      const int kvh = h / group, ctx = pos[t] + 1;
      auto row = [&](const float* pool, int j) {
        return pool + (static_cast<std::int64_t>(table[j / block_size]) * kv_heads + kvh) * block_size * D +
               static_cast<std::int64_t>(j % block_size) * D;
      };
      std::vector<float> score(ctx);
      float mx = -INFINITY;
      for (int j = 0; j < ctx; ++j) {
        score[j] = dot8(qr, row(kpool, j), D) * scale;
        mx = std::max(mx, score[j]);
      }
      float sum = 0;
      for (int j = 0; j < ctx; ++j) {
        score[j] = std::exp(score[j] - mx);
        sum += score[j];
      }
      float* o = out + (static_cast<std::int64_t>(i) * heads + h) * D;
      std::fill(o, o + D, 0.0f);
      for (int j = 0; j < ctx; ++j) {
        const float p = score[j] / sum;
        const float* vr = row(vpool, j);
        for (int d = 0; d < D; ++d) o[d] += p * vr[d];
      }
    }
  }
}

// The same attention by a different route, for pinning the one above: double
// precision throughout, the normalizer summed before any weight is formed.
void oracle_paged_attention_f64(const float* q, long q_stride, const float* kpool, const float* vpool,
                                const int* pos, const int* seq, const int* table_off, const int* tables,
                                const int* tokens, int n, int heads, int kv_heads, int D, int block_size,
                                double scale, double* out) {
  const int group = heads / kv_heads;
#pragma omp parallel for
  for (int i = 0; i < n; ++i) {
    const int t = tokens ? tokens[i] : i;
    const int* table = tables + table_off[seq[t]];
    for (int h = 0; h < heads; ++h) {
      const float* qr = q + static_cast<std::int64_t>(t) * q_stride + h * D;
      const int kvh = h / group, ctx = pos[t] + 1;
      std::vector<double> s(ctx);
      double mx = -INFINITY;
      for (int j = 0; j < ctx; ++j) {
        const int blk = table[j / block_size], slot = j % block_size;
        const float* kr = kpool + ((static_cast<std::int64_t>(blk) * kv_heads + kvh) * block_size + slot) * D;
        double acc = 0;
        for (int d = 0; d < D; ++d) acc += static_cast<double>(qr[d]) * kr[d];
        s[j] = acc * scale;
        mx = std::max(mx, s[j]);
      }
      double* o = out + (static_cast<std::int64_t>(i) * heads + h) * D;
      std::fill(o, o + D, 0.0);
      double z = 0;
      for (int j = 0; j < ctx; ++j) z += std::exp(s[j] - mx);
      for (int j = 0; j < ctx; ++j) {
        const int blk = table[j / block_size], slot = j % block_size;
        const float* vr = vpool + ((static_cast<std::int64_t>(blk) * kv_heads + kvh) * block_size + slot) * D;
        const double p = std::exp(s[j] - mx) / z;
        for (int d = 0; d < D; ++d) o[d] += p * vr[d];
      }
    }
  }
}

// y[t, n] = scale[n] * sum_k W8[n, k] * x[t, k] (+ beta * y0[t, n]) accumulated in
// double: the value the GEMV approximates (gemv_int8_kernel, cuda_kernels.cuh:378-430),
// to within double rounding, far below the fp32 accumulation error under test.
void oracle_gemv_int8(const std::int8_t* w8, const float* scale, const std::uint16_t* x, int T, int K, int N,
                      double beta, const float* y0, double* y) {
#pragma omp parallel for
  for (int n = 0; n < N; ++n) {
    for (int t = 0; t < T; ++t) {
      double acc = 0;
      for (int k = 0; k < K; ++k)
        acc += static_cast<double>(w8[static_cast<std::size_t>(n) * K + k]) * from_f16(x[static_cast<std::size_t>(t) * K + k]);
      double r = acc * scale[n];
      if (beta != 0.0) r += beta * y0[static_cast<std::size_t>(t) * N + n];
      y[static_cast<std::size_t>(t) * N + n] = r;
    }
  }
}

}  // extern "C"
