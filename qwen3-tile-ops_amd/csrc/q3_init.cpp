// Deterministic random-init model image and the per-row int8 weight
// quantiser.
//
// The reference builds its blob from the HF checkpoint (tools/convert_pqwf.py
// :125-220).  That checkpoint cannot be fetched here, so this file writes a
// blob of the same layout from seeded normal draws; everything downstream
// (forward path, oracle, golden vectors) reads weights back from the blob, so
// no two components need to share a random generator.
//
// Generator: z(seed, stream, i) is a Box-Muller standard normal built from a
// counter-based splitmix64 hash, so any element can be produced independently
// and the blob is identical for any thread count.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "q3ops.h"

namespace {

inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
  return mix64(seed ^ mix64(stream ^ 0x632BE59BD9B4E019ull));
}

// Uniform in the open interval (0, 1) with 53 random bits.
inline double uniform_open(uint64_t key, uint64_t i) {
  const uint64_t h = mix64(key + i * 0xD1B54A32D192ED03ull);
  return (static_cast<double>(h >> 11) + 0.5) * 0x1p-53;
}

inline double normal_at(uint64_t key, uint64_t i) {
  const double u1 = uniform_open(key, 2 * i);
  const double u2 = uniform_open(key, 2 * i + 1);
  return std::sqrt(-2.0 * std::log(u1)) *
         std::cos(6.283185307179586476925286766559 * u2);
}

constexpr float kInv127 = 1.0f / 127.0f;  // RN(1/127), kernels/config.h:63

// tools/pqwf.py:72-89 quantize_rows for one row.
void quantize_row(const float *w, size_t cols, int8_t *q, float *scale) {
  float absmax = 0.0f;
  for (size_t c = 0; c < cols; ++c) {
    const float a = std::fabs(w[c]);
    absmax = a > absmax ? a : absmax;
  }
  const float s = absmax * kInv127;
  for (size_t c = 0; c < cols; ++c) {
    const float quot = w[c] / s;
    float r = std::isnan(quot) ? 0.0f : std::nearbyint(quot);
    r = std::min(127.0f, std::max(-127.0f, r));
    q[c] = static_cast<int8_t>(r);
  }
  *scale = s;
}

template <class F>
void parallel_rows(size_t rows, int threads, F &&fn) {
  if (threads <= 1 || rows < 64) {
    fn(size_t(0), rows);
    return;
  }
  std::vector<std::thread> pool;
  const size_t per = (rows + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const size_t r0 = per * t, r1 = std::min(rows, r0 + per);
    if (r0 >= r1) break;
    pool.emplace_back([&fn, r0, r1] { fn(r0, r1); });
  }
  for (auto &th : pool) th.join();
}

// One [rows][cols] weight matrix: row r of stream `stream` uses normal draws
// r*cols .. r*cols+cols-1.
void write_weight(uint64_t seed, uint64_t stream, double std_dev, size_t rows,
                  size_t cols, uint8_t *q_dst, uint8_t *s_dst, int threads) {
  const uint64_t key = stream_key(seed, stream);
  parallel_rows(rows, threads, [&](size_t r0, size_t r1) {
    std::vector<float> row(cols);
    for (size_t r = r0; r < r1; ++r) {
      for (size_t c = 0; c < cols; ++c)
        row[c] = static_cast<float>(std_dev * normal_at(key, r * cols + c));
      float s;
      quantize_row(row.data(), cols,
                   reinterpret_cast<int8_t *>(q_dst + r * cols), &s);
      std::memcpy(s_dst + 4 * r, &s, 4);
    }
  });
}

void write_gain(uint64_t seed, uint64_t stream, double std_dev, size_t n,
                uint8_t *dst) {
  const uint64_t key = stream_key(seed, stream);
  for (size_t i = 0; i < n; ++i) {
    const float g = static_cast<float>(1.0 + std_dev * normal_at(key, i));
    std::memcpy(dst + 4 * i, &g, 4);
  }
}

}  // namespace

extern "C" uint64_t q3_init_stream_id(int layer, int which) {
  if (layer < 0) return 0x100ull + static_cast<uint64_t>(which);
  return 0x10000ull + (static_cast<uint64_t>(layer) << 8) +
         static_cast<uint64_t>(which);
}

extern "C" int q3_init_normal(uint64_t seed, uint64_t stream, uint64_t first,
                              size_t n, double mean, double std_dev,
                              float *out) {
  if (!out && n) return Q3_ERR_ARG;
  const uint64_t key = stream_key(seed, stream);
  for (size_t i = 0; i < n; ++i)
    out[i] = static_cast<float>(mean + std_dev * normal_at(key, first + i));
  return Q3_OK;
}

extern "C" int q3_quantize_rows_host(const float *w, size_t rows, size_t cols,
                                     int8_t *q, float *scale) {
  if ((!w || !q || !scale) && rows) return Q3_ERR_ARG;
  for (size_t r = 0; r < rows; ++r)
    quantize_row(w + r * cols, cols, q + r * cols, scale + r);
  return Q3_OK;
}

extern "C" int q3_init_random_blob(const q3_layout *lay,
                                   const q3_init_params *p, uint8_t *blob,
                                   int threads) {
  if (!lay || !p || !blob) return Q3_ERR_ARG;
  if (p->n_prompt < 0 || p->n_gen < 0 ||
      static_cast<int64_t>(p->n_prompt) + p->n_gen >
          static_cast<int64_t>(lay->max_seq))
    return Q3_ERR_RANGE;
  if (threads <= 0) threads = static_cast<int>(std::thread::hardware_concurrency());
  if (threads <= 0) threads = 1;
  std::memset(blob, 0, static_cast<size_t>(lay->kSCRATCH_END));

  const size_t H = lay->hidden, HD = lay->head_dim, I = lay->inter;
  const size_t V = lay->vocab, QW = size_t(lay->heads) * HD;
  const size_t KW = size_t(lay->kv_heads) * HD, HALF = lay->half;
  const uint64_t seed = p->weight_seed;

  // ids + CTRL (convert_pqwf.py:37-43, 175-177).
  {
    int32_t *ids = reinterpret_cast<int32_t *>(blob + lay->kIDS);
    const int n = p->n_prompt + p->n_gen;
    if (p->ids_seed == 0) {
      for (int i = 0; i < n; ++i) ids[i] = 100 + 10 * i;
    } else {
      const uint64_t key = stream_key(p->ids_seed, 0x1D5);
      for (int i = 0; i < p->n_prompt; ++i)
        ids[i] = static_cast<int32_t>(mix64(key + static_cast<uint64_t>(i)) %
                                      lay->vocab);
    }
    int32_t ctrl[4] = {p->n_prompt, p->n_gen, static_cast<int32_t>(lay->max_seq),
                       p->mode};
    std::memcpy(blob + lay->kCTRL, ctrl, sizeof(ctrl));
  }

  // RoPE tables: f64 angles, rounded to f32 (convert_pqwf.py:46-52).
  {
    float *cs = reinterpret_cast<float *>(blob + lay->kCOS);
    float *sn = reinterpret_cast<float *>(blob + lay->kSIN);
    std::vector<double> inv_freq(HALF);
    for (size_t i = 0; i < HALF; ++i)
      inv_freq[i] = 1.0 / std::pow(p->rope_theta,
                                   static_cast<double>(i) / static_cast<double>(HALF));
    for (size_t pos = 0; pos < lay->max_seq; ++pos)
      for (size_t i = 0; i < HALF; ++i) {
        const double ang = static_cast<double>(pos) * inv_freq[i];
        cs[pos * HALF + i] = static_cast<float>(std::cos(ang));
        sn[pos * HALF + i] = static_cast<float>(std::sin(ang));
      }
  }

  write_gain(seed, q3_init_stream_id(-1, 2), p->gain_std, H, blob + lay->kNF);
  write_weight(seed, q3_init_stream_id(-1, 0), p->weight_std, V, H,
               blob + lay->kEMB, blob + lay->kEMB + V * H, threads);
  write_weight(seed, q3_init_stream_id(-1, 1), p->weight_std, V, H,
               blob + lay->kLM, blob + lay->kLM + V * H, threads);

  struct W {
    int which;
    int64_t q, s;
    size_t rows, cols;
  };
  const W ws[7] = {
      {3, lay->kLQ, lay->kLQ_SCALE, QW, H}, {4, lay->kLK, lay->kLK_SCALE, KW, H},
      {5, lay->kLV, lay->kLV_SCALE, KW, H}, {6, lay->kLO, lay->kLO_SCALE, H, QW},
      {7, lay->kLG, lay->kLG_SCALE, I, H},  {8, lay->kLU, lay->kLU_SCALE, I, H},
      {9, lay->kLD, lay->kLD_SCALE, H, I}};
  for (uint32_t L = 0; L < lay->layers; ++L) {
    const int64_t wbase = static_cast<int64_t>(L) * lay->kLAYERW_STRIDE;
    for (const W &w : ws)
      write_weight(seed, q3_init_stream_id(static_cast<int>(L), w.which),
                   p->weight_std, w.rows, w.cols, blob + w.q + wbase,
                   blob + w.s + wbase, threads);
    const int64_t nbase = static_cast<int64_t>(L) * lay->kLAYERN_STRIDE;
    write_gain(seed, q3_init_stream_id(static_cast<int>(L), 10), p->gain_std, H,
               blob + lay->kN1 + nbase);
    write_gain(seed, q3_init_stream_id(static_cast<int>(L), 11), p->gain_std, HD,
               blob + lay->kNQ + nbase);
    write_gain(seed, q3_init_stream_id(static_cast<int>(L), 12), p->gain_std, HD,
               blob + lay->kNK + nbase);
    write_gain(seed, q3_init_stream_id(static_cast<int>(L), 13), p->gain_std, H,
               blob + lay->kN2 + nbase);
  }
  return Q3_OK;
}
