// CPU ORACLE: test infrastructure only, never product code.
//
// Restatement of the tensor.cx CPU reference arithmetic for the hip hot path
// (matmul, single- and multi-axis sum/max/mean, min/argmax, softmax, RMSNorm,
// LayerNorm, elementwise exp/gelu/silu and broadcast binary arithmetic) and for
// the ops next to it (log/sqrt/abs, clip, topk, attention softmax). Only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
// checker. Each function keeps the reference loop order and rounding exactly:
// built with g++ -O2 -ffp-contract=off (no FMA contraction, no reassociation), it
// is bit-identical to the reference CPU backend. Work is split across threads
// only over independent outputs, which leaves every output's arithmetic
// sequence unchanged.
//
// Pinning: every function is checked against golden vectors made by the
// reference CPU backend itself (tests/golden) and against closed forms in
// tests/test_oracle.py.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

namespace {

using Dim = std::int64_t;

template <typename F>
void parallel_for(Dim count, int threads, F&& body) {
  if (threads <= 1 || count < 2) {
    body(Dim{0}, count);
    return;
  }
  const Dim workers = std::min<Dim>(threads, count);
  std::vector<std::thread> pool;
  pool.reserve(static_cast<std::size_t>(workers));
  for (Dim w = 0; w < workers; ++w) {
    const Dim begin = count * w / workers, end = count * (w + 1) / workers;
    pool.emplace_back([&body, begin, end] { body(begin, end); });
  }
  for (auto& t : pool) t.join();
}

// Bitwise helpers of the reference min/argmax kernel
// (cpp/tensorcx/backends/cpu/cpu_math.cpp:14-20): NaN test on the word and a
// total order in which +0 and -0 compare equal.
bool word_nan(std::uint32_t a, bool fp) { return fp && (a & 0x7fffffffu) > 0x7f800000u; }
bool word_less(std::uint32_t a, std::uint32_t b, bool fp) {
  if (!fp) return static_cast<std::int32_t>(a) < static_cast<std::int32_t>(b);
  if (!(a & 0x7fffffffu)) a = 0;
  if (!(b & 0x7fffffffu)) b = 0;
  const std::uint32_t ka = (a & 0x80000000u) ? ~a : (a ^ 0x80000000u);
  const std::uint32_t kb = (b & 0x80000000u) ? ~b : (b ^ 0x80000000u);
  return ka < kb;
}

}  // namespace

extern "C" {

// cpu_backend.cpp:1251-1276 (cpu::matmul): out[b,i,j] = sum_k a*b in ascending
// k, starting at 0.0f, one multiply and one add per step. The i-k-j loop below
// updates each output's own accumulator in that same ascending k order, so the
// rounding sequence per element is the reference's.
void oracle_matmul_f32(const float* a, const float* b, float* out, Dim batches, Dim m, Dim n,
                       Dim k, const Dim* lhs_offsets, const Dim* rhs_offsets, int threads) {
  const Dim rows = batches * m;
  parallel_for(rows, threads, [&](Dim begin, Dim end) {
    constexpr Dim kRowBlock = 8, kColBlock = 256;
    std::vector<float> acc(static_cast<std::size_t>(kRowBlock * kColBlock));
    for (Dim r0 = begin; r0 < end;) {
      const Dim batch = r0 / m;
      const Dim row0 = r0 % m;
      const Dim rcount = std::min<Dim>({kRowBlock, end - r0, m - row0});
      const float* ab = a + lhs_offsets[batch];
      const float* bb = b + rhs_offsets[batch];
      float* ob = out + batch * m * n;
      for (Dim c0 = 0; c0 < n; c0 += kColBlock) {
        const Dim ccount = std::min<Dim>(kColBlock, n - c0);
        std::fill(acc.begin(), acc.end(), 0.0F);
        for (Dim kk = 0; kk < k; ++kk) {
          const float* brow = bb + kk * n + c0;
          for (Dim r = 0; r < rcount; ++r) {
            const float av = ab[(row0 + r) * k + kk];
            float* accr = acc.data() + r * kColBlock;
            for (Dim c = 0; c < ccount; ++c) {
              const float p = av * brow[c];
              accr[c] = accr[c] + p;
            }
          }
        }
        for (Dim r = 0; r < rcount; ++r)
          std::memcpy(ob + (row0 + r) * n + c0, acc.data() + r * kColBlock,
                      static_cast<std::size_t>(ccount) * sizeof(float));
      }
      r0 += rcount;
    }
  });
}

// Same arithmetic in the reference's literal i-j-k order with column-strided B
// (cpu_backend.cpp:1264-1273). Used to time the reference algorithm itself.
void oracle_matmul_f32_naive(const float* a, const float* b, float* out, Dim m, Dim n, Dim k,
                             Dim row_begin, Dim row_end) {
  for (Dim i = row_begin * n; i < row_end * n; ++i) {
    const Dim col = i % n, row = i / n;
    float sum = 0.0F;
    for (Dim inner = 0; inner < k; ++inner) sum += a[row * k + inner] * b[inner * n + col];
    out[i] = sum;
  }
}

// cpu_backend.cpp:1154-1249 (reduce, single axis). op: 0 sum, 1 max, 2 mean.
// Inputs are [outer, reduce, inner] row-major; outputs [outer, inner].
void oracle_reduce_f32(int op, const float* x, float* out, Dim outer, Dim reduce, Dim inner,
                       int threads) {
  parallel_for(outer * inner, threads, [&](Dim begin, Dim end) {
    for (Dim id = begin; id < end; ++id) {
      const Dim base = (id / inner) * reduce * inner + id % inner;
      if (op == 1) {
        float best = -std::numeric_limits<float>::infinity();
        for (Dim r = 0; r < reduce; ++r) {
          const float v = x[base + r * inner];
          if (std::isnan(v)) {
            best = v;
            break;
          }
          best = std::max(best, v);
        }
        out[id] = best;
      } else {
        if (op == 2 && reduce == 0) {
          out[id] = std::numeric_limits<float>::quiet_NaN();
          continue;
        }
        float sum = 0.0F;
        for (Dim r = 0; r < reduce; ++r) sum += x[base + r * inner];
        out[id] = op == 2 ? sum / static_cast<float>(reduce) : sum;
      }
    }
  });
}

// cpu_backend.cpp:1208-1246: int32 sum wraps modulo 2^32, max is signed.
// op: 0 sum, 1 max.
void oracle_reduce_i32(int op, const std::int32_t* x, std::int32_t* out, Dim outer, Dim reduce,
                       Dim inner, int threads) {
  parallel_for(outer * inner, threads, [&](Dim begin, Dim end) {
    for (Dim id = begin; id < end; ++id) {
      const Dim base = (id / inner) * reduce * inner + id % inner;
      if (op == 1) {
        std::int32_t best = std::numeric_limits<std::int32_t>::min();
        for (Dim r = 0; r < reduce; ++r) best = std::max(best, x[base + r * inner]);
        out[id] = best;
      } else {
        std::uint32_t sum = 0;
        for (Dim r = 0; r < reduce; ++r) sum += static_cast<std::uint32_t>(x[base + r * inner]);
        out[id] = static_cast<std::int32_t>(sum);
      }
    }
  });
}

// cpu_backend.cpp:1102-1153 (reduce over an axis selection). `meta` holds
// extent/stride pairs, kept axes first, then reduced axes, as built by
// make_reduction_plan (shape.cpp:140-173). dtype: 0 float32, 1 int32.
// op: 0 sum, 1 max, 2 mean.
void oracle_reduce_axes(int op, int dtype, const void* x, void* out, const Dim* meta,
                        int outer_rank, int rank, Dim groups, Dim reduction_size, int threads) {
  const auto offset = [&](Dim index, int begin, int end) {
    Dim value = 0;
    for (int axis = end; axis-- > begin;) {
      const Dim extent = meta[2 * axis];
      value += (index % extent) * meta[2 * axis + 1];
      index /= extent;
    }
    return value;
  };
  parallel_for(groups, threads, [&](Dim begin, Dim end) {
    for (Dim g = begin; g < end; ++g) {
      const Dim base = offset(g, 0, outer_rank);
      if (dtype == 0) {
        const float* xf = static_cast<const float*>(x);
        float value = op == 1 ? -std::numeric_limits<float>::infinity() : 0.0F;
        for (Dim r = 0; r < reduction_size; ++r) {
          const float item = xf[base + offset(r, outer_rank, rank)];
          if (op == 1) {
            if (std::isnan(item)) {
              value = item;
              break;
            }
            value = std::max(value, item);
          } else {
            value += item;
          }
        }
        if (op == 2)
          value = reduction_size ? value / static_cast<float>(reduction_size)
                                 : std::numeric_limits<float>::quiet_NaN();
        static_cast<float*>(out)[g] = value;
      } else {
        const std::int32_t* xi = static_cast<const std::int32_t*>(x);
        std::uint32_t sum = 0;
        std::int32_t best = std::numeric_limits<std::int32_t>::min();
        for (Dim r = 0; r < reduction_size; ++r) {
          const std::int32_t item = xi[base + offset(r, outer_rank, rank)];
          if (op == 1)
            best = std::max(best, item);
          else
            sum += static_cast<std::uint32_t>(item);
        }
        static_cast<std::int32_t*>(out)[g] = op == 1 ? best : static_cast<std::int32_t>(sum);
      }
    }
  });
}

// cpu_math.cpp:48-54 (codes 3 min, 4 argmax). `meta` is the reduction plan's
// extent/stride list over all `rank` axes (kept first, reduced last); element
// j of group g is at mapped(g*reduce + j). The first element seeds the best; a
// NaN best is sticky; a later element replaces it when it is NaN or strictly
// better, so ties keep the lowest index. out is float32/int32 words for min,
// int32 indices for argmax.
void oracle_argext(int code, int dtype, const std::uint32_t* x, std::uint32_t* out,
                   const Dim* meta, int rank, Dim groups, Dim reduce, int threads) {
  const bool fp = dtype == 0;
  const auto mapped = [&](Dim i) {
    Dim source = 0;
    for (int a = rank; a-- > 0;) {
      source += i % meta[2 * a] * meta[2 * a + 1];
      i /= meta[2 * a];
    }
    return source;
  };
  parallel_for(groups, threads, [&](Dim begin, Dim end) {
    for (Dim g = begin; g < end; ++g) {
      std::uint32_t best = x[mapped(g * reduce)];
      Dim index = 0;
      for (Dim j = 1; j < reduce; ++j) {
        const std::uint32_t a = x[mapped(g * reduce + j)];
        if (!word_nan(best, fp) &&
            (word_nan(a, fp) || (code == 3 ? word_less(a, best, fp) : word_less(best, a, fp)))) {
          best = a;
          index = j;
        }
      }
      out[g] = code == 4 ? static_cast<std::uint32_t>(index) : best;
    }
  });
}

// cpu_backend.cpp:125-155 (compute_softmax): NaN-first max, sequential sum of
// exp(x - max), then exp recomputed and divided.
void oracle_softmax(const float* x, float* out, Dim outer, Dim reduce, Dim inner, int threads) {
  parallel_for(outer * inner, threads, [&](Dim begin, Dim end) {
    for (Dim id = begin; id < end; ++id) {
      const Dim base = (id / inner) * reduce * inner + id % inner;
      float m = -std::numeric_limits<float>::infinity();
      for (Dim r = 0; r < reduce; ++r) {
        const float v = x[base + r * inner];
        if (std::isnan(v)) {
          m = v;
          break;
        }
        m = std::max(m, v);
      }
      float denom = 0.0F;
      for (Dim r = 0; r < reduce; ++r) denom += std::exp(x[base + r * inner] - m);
      for (Dim r = 0; r < reduce; ++r) {
        const Dim i = base + r * inner;
        out[i] = std::exp(x[i] - m) / denom;
      }
    }
  });
}

// cpu_backend.cpp:157-183 (compute_rmsnorm).
void oracle_rmsnorm(const float* x, float* out, Dim outer, Dim reduce, Dim inner, float eps,
                    int threads) {
  parallel_for(outer * inner, threads, [&](Dim begin, Dim end) {
    for (Dim id = begin; id < end; ++id) {
      const Dim base = (id / inner) * reduce * inner + id % inner;
      float ss = 0.0F;
      for (Dim r = 0; r < reduce; ++r) {
        const float v = x[base + r * inner];
        ss += v * v;
      }
      const float scale = 1.0F / std::sqrt((ss / static_cast<float>(reduce)) + eps);
      for (Dim r = 0; r < reduce; ++r) {
        const Dim i = base + r * inner;
        out[i] = x[i] * scale;
      }
    }
  });
}

// cpu_backend.cpp:185-240 (compute_layernorm): all-equal finite rows give 0
// (NaN when eps is 0); a zero variance+eps gives NaN.
void oracle_layernorm(const float* x, float* out, Dim outer, Dim reduce, Dim inner, float eps,
                      int threads) {
  parallel_for(outer * inner, threads, [&](Dim begin, Dim end) {
    for (Dim id = begin; id < end; ++id) {
      const Dim base = (id / inner) * reduce * inner + id % inner;
      float sum = 0.0F;
      const float first = x[base];
      bool all_equal = true;
      for (Dim r = 0; r < reduce; ++r) {
        const float v = x[base + r * inner];
        sum += v;
        all_equal = all_equal && v == first;
      }
      if (all_equal && std::isfinite(first)) {
        const float v = eps == 0.0F ? std::numeric_limits<float>::quiet_NaN() : 0.0F;
        for (Dim r = 0; r < reduce; ++r) out[base + r * inner] = v;
        continue;
      }
      const float mean = sum / static_cast<float>(reduce);
      float ssd = 0.0F;
      for (Dim r = 0; r < reduce; ++r) {
        const float d = x[base + r * inner] - mean;
        ssd += d * d;
      }
      const float denom = ssd / static_cast<float>(reduce) + eps;
      if (denom == 0.0F) {
        for (Dim r = 0; r < reduce; ++r) out[base + r * inner] = std::numeric_limits<float>::quiet_NaN();
        continue;
      }
      const float scale = 1.0F / std::sqrt(denom);
      for (Dim r = 0; r < reduce; ++r) {
        const Dim i = base + r * inner;
        out[i] = (x[i] - mean) * scale;
      }
    }
  });
}

// cpu_backend.cpp:1000-1010 (execute_unary tail). op: 0 exp, 1 gelu, 2 silu.
void oracle_unary(int op, const float* x, float* out, Dim n, int threads) {
  constexpr float kTanh = 0.7978845608028654F;
  constexpr float kCubic = 0.044715F;
  parallel_for(n, threads, [&](Dim begin, Dim end) {
    for (Dim i = begin; i < end; ++i) {
      const float v = x[i];
      if (op == 0) {
        out[i] = std::exp(v);
      } else if (op == 1) {
        const float in = kTanh * (v + kCubic * v * v * v);
        out[i] = 0.5F * v * (1.0F + std::tanh(in));
      } else {
        out[i] = v / (1.0F + std::exp(-v));
      }
    }
  });
}

// cpu_backend.cpp:1014-1097 (execute_binary) over a broadcast plan
// (shape.cpp:202-229). op: 0 add, 1 subtract, 2 multiply, 3 divide.
// dtype 0 float32; dtype 1 int32 computed in uint32 (wrapping).
void oracle_binary(int op, int dtype, const void* lhs, const void* rhs, void* out,
                   const Dim* out_shape, const Dim* lhs_strides, const Dim* rhs_strides, int rank,
                   Dim count, int threads) {
  parallel_for(count, threads, [&](Dim begin, Dim end) {
    for (Dim i = begin; i < end; ++i) {
      Dim index = i, left = 0, right = 0;
      for (int axis = rank; axis-- > 0;) {
        const Dim c = index % out_shape[axis];
        index /= out_shape[axis];
        left += c * lhs_strides[axis];
        right += c * rhs_strides[axis];
      }
      if (dtype == 0) {
        const float a = static_cast<const float*>(lhs)[left];
        const float b = static_cast<const float*>(rhs)[right];
        float r = 0.0F;
        switch (op) {
          case 0: r = a + b; break;
          case 1: r = a - b; break;
          case 2: r = a * b; break;
          default: r = a / b; break;
        }
        static_cast<float*>(out)[i] = r;
      } else {
        const auto a = static_cast<std::uint32_t>(static_cast<const std::int32_t*>(lhs)[left]);
        const auto b = static_cast<std::uint32_t>(static_cast<const std::int32_t*>(rhs)[right]);
        std::uint32_t r = 0;
        switch (op) {
          case 0: r = a + b; break;
          case 1: r = a - b; break;
          default: r = a * b; break;
        }
        static_cast<std::int32_t*>(out)[i] = static_cast<std::int32_t>(r);
      }
    }
  });
}

// cpu_math.cpp:40-44: log and sqrt through the float overloads of std::log and
// std::sqrt; abs clears the sign bit (float32) or negates in uint32 (int32, so
// INT32_MIN stays INT32_MIN). code: 0 log, 1 sqrt, 2 abs.
void oracle_math_unary(int code, int dtype, const std::uint32_t* x, std::uint32_t* out, Dim n,
                       int threads) {
  const bool fp = dtype == 0;
  parallel_for(n, threads, [&](Dim begin, Dim end) {
    for (Dim i = begin; i < end; ++i) {
      std::uint32_t a = x[i];
      if (code == 2) {
        a = fp ? (a & 0x7fffffffu) : ((a & 0x80000000u) ? 0u - a : a);
      } else {
        float f;
        std::memcpy(&f, &a, 4);
        f = code == 0 ? std::log(f) : std::sqrt(f);
        std::memcpy(&a, &f, 4);
      }
      out[i] = a;
    }
  });
}

// cpu_math.cpp:45-50: clip(x, lo, hi) over a three-way broadcast. A NaN x
// stays; otherwise a NaN bound, or a bound the value does not exceed (under
// the +0 == -0 total order), replaces it; lo first, then hi.
// strides holds rank strides for x, then lo, then hi.
void oracle_clip(int dtype, const std::uint32_t* x, const std::uint32_t* lo, const std::uint32_t* hi,
                 std::uint32_t* out, const Dim* shape, const Dim* strides, int rank, Dim count,
                 int threads) {
  const bool fp = dtype == 0;
  parallel_for(count, threads, [&](Dim begin, Dim end) {
    for (Dim i = begin; i < end; ++i) {
      Dim flat = i, ox = 0, ol = 0, oh = 0;
      for (int a = rank; a-- > 0;) {
        const Dim c = flat % shape[a];
        flat /= shape[a];
        ox += c * strides[a];
        ol += c * strides[rank + a];
        oh += c * strides[2 * rank + a];
      }
      std::uint32_t v = x[ox];
      const std::uint32_t l = lo[ol], h = hi[oh];
      if (!word_nan(v, fp)) v = (word_nan(l, fp) || !word_less(l, v, fp)) ? l : v;
      if (!word_nan(v, fp)) v = (word_nan(h, fp) || !word_less(v, h, fp)) ? h : v;
      out[i] = v;
    }
  });
}

// cpu_math.cpp:57-67: top-k along an axis (outer, reduce, inner). Order: NaN
// first when largest (last otherwise), then by value under the +0 == -0 total
// order, then by lower index. sorted == 0 lists the chosen k by index.
void oracle_topk(int dtype, int largest, int sorted, const std::uint32_t* x, std::uint32_t* values,
                 std::int32_t* indices, Dim outer, Dim reduce, Dim inner, Dim k, int threads) {
  const bool fp = dtype == 0;
  parallel_for(outer * inner, threads, [&](Dim begin, Dim end) {
    std::vector<std::int32_t> order(static_cast<std::size_t>(reduce));
    for (Dim g = begin; g < end; ++g) {
      const Dim base = (g / inner) * reduce * inner + g % inner;
      for (Dim j = 0; j < reduce; ++j) order[static_cast<std::size_t>(j)] = static_cast<std::int32_t>(j);
      const auto before = [&](std::int32_t ia, std::int32_t ib) {
        const std::uint32_t a = x[base + ia * inner], b = x[base + ib * inner];
        const bool an = word_nan(a, fp), bn = word_nan(b, fp);
        if (an != bn) return largest ? an : bn;
        if (!an && (word_less(a, b, fp) || word_less(b, a, fp)))
          return largest ? word_less(b, a, fp) : word_less(a, b, fp);
        return ia < ib;
      };
      std::partial_sort(order.begin(), order.begin() + k, order.end(), before);
      if (!sorted) std::sort(order.begin(), order.begin() + k);
      for (Dim j = 0; j < k; ++j) {
        const Dim dest = (g / inner) * k * inner + j * inner + g % inner;
        values[dest] = x[base + order[static_cast<std::size_t>(j)] * inner];
        indices[dest] = order[static_cast<std::size_t>(j)];
      }
    }
  });
}

// cpu_inference.cpp:22-47: attention softmax over the last axis of `shape`.
// The score of (row, col) is -inf when causal and col > row % rows_per_matrix,
// or when a bool mask (mask_kind 1) is false; an additive mask (mask_kind 2)
// of -inf gives -inf; otherwise scores * scale + bias, rounded separately.
// NaN-first maximum; a row whose maximum is -inf is all zeros; else
// exp(s - max) / sequential sum. strides: rank strides for scores, then mask.
void oracle_attention_softmax(const float* scores, const void* mask, int mask_kind, float* out,
                              const Dim* shape, const Dim* strides, int rank, Dim rows, Dim columns,
                              float scale, int causal, int threads) {
  const Dim per_matrix = shape[rank - 2];
  parallel_for(rows, threads, [&](Dim begin, Dim end) {
    for (Dim row = begin; row < end; ++row) {
      const Dim query = row % per_matrix;
      const auto offset = [&](Dim i, int arg) {
        Dim result = 0;
        for (int a = rank; a-- > 0;) {
          result += i % shape[a] * strides[arg * rank + a];
          i /= shape[a];
        }
        return result;
      };
      const auto score = [&](Dim col) -> float {
        const Dim i = row * columns + col;
        const float neg_inf = -std::numeric_limits<float>::infinity();
        if (causal && col > query) return neg_inf;
        if (mask_kind == 1 && !static_cast<const std::uint8_t*>(mask)[offset(i, 1)]) return neg_inf;
        const float bias = mask_kind == 2 ? static_cast<const float*>(mask)[offset(i, 1)] : 0.0F;
        if (bias == neg_inf) return bias;
        const float product = scores[offset(i, 0)] * scale;
        return product + bias;
      };
      float maximum = -std::numeric_limits<float>::infinity();
      for (Dim col = 0; col < columns; ++col) {
        const float v = score(col);
        if (std::isnan(v)) {
          maximum = v;
          break;
        }
        maximum = maximum < v ? v : maximum;
      }
      float* o = out + row * columns;
      if (maximum == -std::numeric_limits<float>::infinity()) {
        for (Dim col = 0; col < columns; ++col) o[col] = 0.0F;
        continue;
      }
      float total = 0.0F;
      for (Dim col = 0; col < columns; ++col) total += std::exp(score(col) - maximum);
      for (Dim col = 0; col < columns; ++col) o[col] = std::exp(score(col) - maximum) / total;
    }
  });
}

}  // extern "C"
