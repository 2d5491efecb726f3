// pxs oracle: a CPU restatement of the reference sparse-voxel path.
//
// TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py load this library, and only as the reference
// that results are compared with.
// The shipped library (pixal3d.cpp_amd/) never links, loads or calls it.
//
// Every function restates the reference algorithm with the reference's loop
// and accumulation order, so that compiled with the reference's Release flags
// (-O3, OpenMP, no -ffast-math, no -march) it rounds identically.  Each
// function names the reference file:line it follows.  Two functions have no
// reference counterpart and define this build's contract instead; they are
// marked "contract" below (strided conv features, window partition).
//
// Pinning (what checks each function beyond its own formula):
//   orc_sparse_valid           error strings + first-error order vs the compiled
//                              reference (oracle/_ref) on planted faults
//   orc_neighbor_map_k3        brute-force sorted-key search (independent of
//                              the reference's unordered_map); invariants
//                              idx[13][p]=p and idx[k][p]=q <=> idx[26-k][q]=p
//   orc_neighbor_pairs         derived from the dense map; counts sum to P
//   orc_subm_conv3d            bit-exact vs oracle/_ref and the reference KAT;
//                              closed form (centre identity => out = in + bias)
//   orc_linear, orc_layer_norm, orc_mh_rms_norm, orc_rope, orc_sdpa,
//   orc_cross_attention, orc_channel_to_spatial, orc_downsample_mean
//                              bit-exact vs oracle/_ref and the reference KATs;
//                              closed forms in tests (identical keys => mean(V))
//   orc_transformer_block      bit-exact vs oracle/_ref and the reference block KAT
//   orc_timestep_embed_mlp     bit-exact vs oracle/_ref
//   orc_slat_flow_forward      composition of pinned pieces; parity unpinned as a
//                              whole (src/slat_flow.cpp needs ggml to build)
//   orc_convnext_block, orc_resblock_c2s
//                              composition of pinned pieces; parity unpinned as a
//                              whole (src/slat_decoder.cpp needs ggml to build)
//   orc_downsample_coords_s2   topology = orc_downsample_mean's coordinates
//   orc_sparse_conv3d_s2       contract; pinned by the invariant W_c = I,
//                              bias = 0 => out = count * mean-pool
//   orc_window_partition       contract; pinned by brute-force invariants in tests
//                              (window membership, stable order, permutation)
//   orc_flow_schedule, orc_flow_guidance, orc_flow_euler_sample
//                              bit-exact vs oracle/_ref (the reference's
//                              src/flow_sampler.cpp compiled where it lies, driven
//                              with the same velocity callback); closed forms in
//                              tests (zero velocity keeps the state; guidance 1 or
//                              0 selects one branch; constant velocity v moves the
//                              state by -v in total)

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <numeric>
#include <vector>

#if defined(_OPENMP)
#include <omp.h>
#endif

namespace {

// A voxel key that orders lexicographically by (batch, x, y, z).  Used for
// the brute-force neighbor search; coordinates are non-negative and below 2^15
// per axis, batch below 2^15 (checked by the callers' validation).
inline uint64_t pack_key(int32_t b, int32_t x, int32_t y, int32_t z) {
    return (static_cast<uint64_t>(static_cast<uint32_t>(b) & 0xFFFFu) << 48) |
           (static_cast<uint64_t>(static_cast<uint32_t>(x) & 0xFFFFu) << 32) |
           (static_cast<uint64_t>(static_cast<uint32_t>(y) & 0xFFFFu) << 16) |
           static_cast<uint64_t>(static_cast<uint32_t>(z) & 0xFFFFu);
}

struct SortedKeys {
    std::vector<uint64_t> keys;
    std::vector<int32_t> rows;
};

SortedKeys sort_keys(const int32_t * coords, int64_t n) {
    std::vector<std::pair<uint64_t, int32_t>> kv(static_cast<size_t>(n));
    for (int64_t p = 0; p < n; ++p) {
        const int32_t * c = coords + p * 4;
        kv[p] = {pack_key(c[0], c[1], c[2], c[3]), static_cast<int32_t>(p)};
    }
    std::sort(kv.begin(), kv.end());
    SortedKeys s;
    s.keys.resize(kv.size());
    s.rows.resize(kv.size());
    for (size_t i = 0; i < kv.size(); ++i) {
        s.keys[i] = kv[i].first;
        s.rows[i] = kv[i].second;
    }
    return s;
}

// First row holding the key, or -1.
int32_t find_key(const SortedKeys & s, int32_t b, int32_t x, int32_t y, int32_t z) {
    if (x < 0 || y < 0 || z < 0) return -1;
    const uint64_t key = pack_key(b, x, y, z);
    auto it = std::lower_bound(s.keys.begin(), s.keys.end(), key);
    if (it == s.keys.end() || *it != key) return -1;
    return s.rows[static_cast<size_t>(it - s.keys.begin())];
}

float silu_reciprocal_form(float v) {
    // src/flow.cpp:83-88 and src/slat_decoder.cpp:68-78: v * (1 / (1 + e^-v)).
    const float sigmoid = 1.0f / (1.0f + std::exp(-v));
    return v * sigmoid;
}

float silu_branch_form(float v) {
    // src/slat_flow.cpp:79-83: the two-branch stable form.
    if (v >= 0.0f) return v / (1.0f + std::exp(-v));
    const float e = std::exp(v);
    return v * e / (1.0f + e);
}

float gelu_tanh(float v) {
    // src/sparse_transformer.cpp:123-134.
    const float k = 0.7978845608028654f;
    const float cubic = v * v * v;
    return 0.5f * v * (1.0f + std::tanh(k * (v + 0.044715f * cubic)));
}

} // namespace

extern "C" {

// ---------------------------------------------------------------------------
// a1: SparseTensorF32::valid (src/sparse.cpp:241-335).
// Returns 0 when valid, else a code naming the reference's message:
//   1 "invalid sparse tensor shape"
//   3 "sparse feature count does not match coordinates"
//   4 "sparse coordinate is outside its shape"
//   5 "sparse coordinates contain a duplicate point"
//   6 "sparse coordinates must be contiguous by batch"
//   7 "sparse features contain a non-finite value"
// *bad_point receives the row at which the scan stopped (-1 for 0/1/3).
// feats_count is the number of floats in feats (n*channels when consistent).
int orc_sparse_valid(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                     int sz, const float * feats, int64_t feats_count, int channels,
                     int64_t * bad_point) {
    *bad_point = -1;
    if (batch_size <= 0 || channels <= 0 || sx <= 0 || sy <= 0 || sz <= 0) return 1;
    if (feats_count != n * static_cast<int64_t>(channels)) return 3;
    // Duplicates: the reference's hash-set insertion fails at the first row
    // whose key appeared at an earlier row.  Sorting (key, row) pairs gives
    // each key's first row; every later row of that key is a duplicate.
    std::vector<std::pair<uint64_t, int64_t>> kv(static_cast<size_t>(n));
    for (int64_t p = 0; p < n; ++p) {
        const int32_t * c = coords + p * 4;
        kv[p] = {pack_key(c[0], c[1], c[2], c[3]), p};
    }
    std::sort(kv.begin(), kv.end());
    std::vector<char> duplicate(static_cast<size_t>(n), 0);
    for (size_t i = 1; i < kv.size(); ++i) {
        if (kv[i].first == kv[i - 1].first) duplicate[kv[i].second] = 1;
    }
    for (int64_t p = 0; p < n; ++p) {
        const int32_t * c = coords + p * 4;
        if (c[0] < 0 || c[0] >= batch_size || c[1] < 0 || c[1] >= sx || c[2] < 0 ||
            c[2] >= sy || c[3] < 0 || c[3] >= sz) {
            *bad_point = p;
            return 4;
        }
        if (duplicate[p]) {
            *bad_point = p;
            return 5;
        }
        if (p > 0 && coords[(p - 1) * 4] > c[0]) {
            *bad_point = p;
            return 6;
        }
        for (int ch = 0; ch < channels; ++ch) {
            if (!std::isfinite(feats[p * channels + ch])) {
                *bad_point = p;
                return 7;
            }
        }
    }
    return 0;
}

// ---------------------------------------------------------------------------
// a2: neighbor gather map (src/slat_decoder.cpp:609-668; offsets as in
// src/sparse.cpp:1030-1035).  idx[k * n + p] = row of the voxel at
// (b, x+kd-1, y+kh-1, z+kw-1), k = kd*9 + kh*3 + kw, or n when absent.
// Brute force over sorted keys, independent of the reference's hash.
void orc_neighbor_map_k3(const int32_t * coords, int64_t n, int32_t * idx) {
    const SortedKeys s = sort_keys(coords, n);
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < n; ++p) {
        const int32_t * c = coords + p * 4;
        for (int k = 0; k < 27; ++k) {
            const int kd = k / 9, kh = (k / 3) % 3, kw = k % 3;
            const int32_t row = find_key(s, c[0], c[1] + kd - 1, c[2] + kh - 1, c[3] + kw - 1);
            idx[static_cast<int64_t>(k) * n + p] = row < 0 ? static_cast<int32_t>(n) : row;
        }
    }
}

// Compacted per-offset pair lists from a dense map: for each k ascending, the
// (input row, output row) pairs with output rows ascending.  offsets[28] are
// the list boundaries.  pair_in/pair_out may be null to count only.
void orc_neighbor_pairs(const int32_t * idx, int64_t n, int32_t * pair_in, int32_t * pair_out,
                        int64_t * offsets) {
    int64_t total = 0;
    for (int k = 0; k < 27; ++k) {
        offsets[k] = total;
        for (int64_t p = 0; p < n; ++p) {
            const int32_t in = idx[static_cast<int64_t>(k) * n + p];
            if (in == n) continue;
            if (pair_in) pair_in[total] = in;
            if (pair_out) pair_out[total] = static_cast<int32_t>(p);
            ++total;
        }
    }
    offsets[27] = total;
}

// ---------------------------------------------------------------------------
// a3: sparse_submanifold_conv3d (src/sparse.cpp:999-1055).  Weight [27, cout,
// cin].  Per output row: for k ascending, for each out channel the dot
// product over in ascending (starting from 0) is added to the accumulator
// (which starts at 0); bias is added last.
void orc_subm_conv3d(const int32_t * coords, int64_t n, const float * feats, int cin,
                     const float * weight, const float * bias, int cout, float * out) {
    std::vector<int32_t> idx(static_cast<size_t>(27 * n));
    orc_neighbor_map_k3(coords, n, idx.data());
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < n; ++p) {
        float * dst = out + p * cout;
        for (int o = 0; o < cout; ++o) dst[o] = 0.0f;
        for (int k = 0; k < 27; ++k) {
            const int32_t src_row = idx[static_cast<int64_t>(k) * n + p];
            if (src_row == n) continue;
            const float * src = feats + static_cast<int64_t>(src_row) * cin;
            const float * kernel = weight + static_cast<int64_t>(k) * cout * cin;
            for (int o = 0; o < cout; ++o) {
                const float * wrow = kernel + static_cast<int64_t>(o) * cin;
                float acc = 0.0f;
                for (int i = 0; i < cin; ++i) acc += wrow[i] * src[i];
                dst[o] += acc;
            }
        }
        for (int o = 0; o < cout; ++o) dst[o] += bias[o];
    }
}

// ---------------------------------------------------------------------------
// a4 (contract): stride-2 sparse conv with a 2x2x2 kernel.
// Output topology = unique (b, x/2, y/2, z/2) in lexicographic order, the
// same coordinates sparse_downsample_mean produces (src/sparse.cpp:553-593).
// Returns the number of output rows; out_coords must hold 4*n ints and
// child_rows 8*n ints (child c = (x&1) + 2*(y&1) + 4*(z&1), -1 when absent).
int64_t orc_downsample_coords_s2(const int32_t * coords, int64_t n, int32_t * out_coords,
                                 int32_t * child_rows) {
    std::vector<std::pair<uint64_t, int64_t>> kv(static_cast<size_t>(n));
    for (int64_t p = 0; p < n; ++p) {
        const int32_t * c = coords + p * 4;
        kv[p] = {pack_key(c[0], c[1] / 2, c[2] / 2, c[3] / 2), p};
    }
    std::sort(kv.begin(), kv.end());
    int64_t m = -1;
    uint64_t last = ~0ull;
    for (size_t i = 0; i < kv.size(); ++i) {
        if (i == 0 || kv[i].first != last) {
            ++m;
            last = kv[i].first;
            const int32_t * c = coords + kv[i].second * 4;
            out_coords[m * 4 + 0] = c[0];
            out_coords[m * 4 + 1] = c[1] / 2;
            out_coords[m * 4 + 2] = c[2] / 2;
            out_coords[m * 4 + 3] = c[3] / 2;
            for (int j = 0; j < 8; ++j) child_rows[m * 8 + j] = -1;
        }
        const int32_t * c = coords + kv[i].second * 4;
        const int child = (c[1] & 1) + 2 * (c[2] & 1) + 4 * (c[3] & 1);
        child_rows[m * 8 + child] = static_cast<int32_t>(kv[i].second);
    }
    return m + 1;
}

// out[q] = sum over present children c ascending of W_c . x[child] + bias,
// each dot product over in ascending from 0, bias last (the same order as
// orc_subm_conv3d).  Weight [8, cout, cin].
void orc_sparse_conv3d_s2(const int32_t * child_rows, int64_t m, const float * feats, int cin,
                          const float * weight, const float * bias, int cout, float * out) {
#pragma omp parallel for schedule(static)
    for (int64_t q = 0; q < m; ++q) {
        float * dst = out + q * cout;
        for (int o = 0; o < cout; ++o) dst[o] = 0.0f;
        for (int c = 0; c < 8; ++c) {
            const int32_t row = child_rows[q * 8 + c];
            if (row < 0) continue;
            const float * src = feats + static_cast<int64_t>(row) * cin;
            const float * kernel = weight + static_cast<int64_t>(c) * cout * cin;
            for (int o = 0; o < cout; ++o) {
                const float * wrow = kernel + static_cast<int64_t>(o) * cin;
                float acc = 0.0f;
                for (int i = 0; i < cin; ++i) acc += wrow[i] * src[i];
                dst[o] += acc;
            }
        }
        for (int o = 0; o < cout; ++o) dst[o] += bias[o];
    }
}

// ---------------------------------------------------------------------------
// a15: sparse_downsample_mean (src/sparse.cpp:536-602).  Groups rows by
// (b, x/f, y/f, z/f); each group's sum runs over its rows in input order, then
// is divided by the count; groups are emitted in lexicographic order.
// Returns the group count.
int64_t orc_downsample_mean(const int32_t * coords, int64_t n, const float * feats, int channels,
                            int factor, int32_t * out_coords, float * out_feats) {
    std::vector<std::pair<uint64_t, int64_t>> kv(static_cast<size_t>(n));
    for (int64_t p = 0; p < n; ++p) {
        const int32_t * c = coords + p * 4;
        kv[p] = {pack_key(c[0], c[1] / factor, c[2] / factor, c[3] / factor), p};
    }
    // Stable by row within a key so each group's sum runs in input order.
    std::sort(kv.begin(), kv.end());
    int64_t m = 0;
    size_t i = 0;
    std::vector<float> sum(static_cast<size_t>(channels));
    while (i < kv.size()) {
        size_t j = i;
        std::fill(sum.begin(), sum.end(), 0.0f);
        while (j < kv.size() && kv[j].first == kv[i].first) {
            const float * src = feats + kv[j].second * channels;
            for (int ch = 0; ch < channels; ++ch) sum[ch] += src[ch];
            ++j;
        }
        const int32_t * c = coords + kv[i].second * 4;
        out_coords[m * 4 + 0] = c[0];
        out_coords[m * 4 + 1] = c[1] / factor;
        out_coords[m * 4 + 2] = c[2] / factor;
        out_coords[m * 4 + 3] = c[3] / factor;
        const float count = static_cast<float>(j - i);
        for (int ch = 0; ch < channels; ++ch) out_feats[m * channels + ch] = sum[ch] / count;
        ++m;
        i = j;
    }
    return m;
}

// ---------------------------------------------------------------------------
// a5: sparse_channel_to_spatial (src/sparse.cpp:604-702) with factor 2 or any
// positive factor.  subdivision (may be null) is [n, factor^3]; values > 0
// select children.  Output is parent-major, child ascending; child c has
// x bit c % f, y bit (c / f) % f, z bit c / f^2.  Returns the output rows.
int64_t orc_channel_to_spatial(const int32_t * coords, int64_t n, const float * feats,
                               int channels, int factor, const float * subdivision,
                               int32_t * out_coords, float * out_feats) {
    const int children = factor * factor * factor;
    const int out_ch = channels / children;
    int64_t m = 0;
    for (int64_t p = 0; p < n; ++p) {
        const int32_t * c = coords + p * 4;
        for (int child = 0; child < children; ++child) {
            if (subdivision && subdivision[p * children + child] <= 0.0f) continue;
            const int cx = child % factor;
            const int cy = (child / factor) % factor;
            const int cz = child / (factor * factor);
            if (out_coords) {
                out_coords[m * 4 + 0] = c[0];
                out_coords[m * 4 + 1] = c[1] * factor + cx;
                out_coords[m * 4 + 2] = c[2] * factor + cy;
                out_coords[m * 4 + 3] = c[3] * factor + cz;
            }
            if (out_feats) {
                std::memcpy(out_feats + m * out_ch, feats + p * channels + child * out_ch,
                            sizeof(float) * static_cast<size_t>(out_ch));
            }
            ++m;
        }
    }
    return m;
}

// ---------------------------------------------------------------------------
// a6: sparse_linear / varlen_linear / row_linear (src/sparse.cpp:434-447,
// 476-486; src/slat_flow.cpp:85-111).  Bias first, then in ascending.
namespace {
inline void linear_row(const float * src, int cin, const float * weight, const float * bias,
                       int cout, float * dst) {
    for (int o = 0; o < cout; ++o) {
        float acc = bias[o];
        const float * wrow = weight + static_cast<int64_t>(o) * cin;
        for (int i = 0; i < cin; ++i) acc += wrow[i] * src[i];
        dst[o] = acc;
    }
}
}  // namespace

void orc_linear(const float * x, int64_t rows, int cin, const float * weight, const float * bias,
                int cout, float * y) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) linear_row(x + r * cin, cin, weight, bias, cout, y + r * cout);
}

namespace {
// orc_linear on the listed rows only (all rows when `rows` is null).  Every
// output element is computed alone, in the same order, so a listed row equals
// orc_linear's bit for bit; unlisted rows of y are left as they are.
void linear_on_rows(const float * x, int64_t n, int cin, const float * weight, const float * bias,
                    int cout, float * y, const int64_t * rows, int64_t row_count) {
    if (!rows) {
        orc_linear(x, n, cin, weight, bias, cout, y);
        return;
    }
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < row_count; ++i) {
        const int64_t r = rows[i];
        linear_row(x + r * cin, cin, weight, bias, cout, y + r * cout);
    }
}
}  // namespace

// ---------------------------------------------------------------------------
// a12: sparse_layer_norm (src/sparse.cpp:490-534): two-pass mean/variance.
void orc_layer_norm(const float * x, int64_t rows, int channels, float eps, const float * gamma,
                    const float * beta, float * y) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float * src = x + r * channels;
        float * dst = y + r * channels;
        float mean = 0.0f;
        for (int c = 0; c < channels; ++c) mean += src[c];
        mean /= static_cast<float>(channels);
        float var = 0.0f;
        for (int c = 0; c < channels; ++c) {
            const float d = src[c] - mean;
            var += d * d;
        }
        var /= static_cast<float>(channels);
        const float inv = 1.0f / std::sqrt(var + eps);
        for (int c = 0; c < channels; ++c) {
            float v = (src[c] - mean) * inv;
            if (gamma) v = v * gamma[c] + beta[c];
            dst[c] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// a10: sparse_multihead_rms_norm / varlen_multihead_rms_norm
// (src/sparse.cpp:919-954, 956-997).
void orc_mh_rms_norm(const float * x, int64_t rows, int heads, int head_dim, const float * gamma,
                     float * y) {
    const int channels = heads * head_dim;
    const float mult = std::sqrt(static_cast<float>(head_dim));
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float * src = x + r * channels;
        float * dst = y + r * channels;
        for (int h = 0; h < heads; ++h) {
            const int off = h * head_dim;
            float sq = 0.0f;
            for (int d = 0; d < head_dim; ++d) sq += src[off + d] * src[off + d];
            const float inv = 1.0f / std::max(std::sqrt(sq), 1e-12f);
            for (int d = 0; d < head_dim; ++d) {
                dst[off + d] = src[off + d] * inv * mult * gamma[off + d];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// a11: sparse_rotary_position_embedding (src/sparse.cpp:861-917).
void orc_rope(const int32_t * coords, const float * x, int64_t rows, int heads, int head_dim,
              float freq_min, float freq_base, float * y) {
    const int channels = heads * head_dim;
    const int pairs = head_dim / 2;
    const int fdim = pairs / 3;
    std::vector<float> freqs(static_cast<size_t>(std::max(fdim, 0)));
    for (int i = 0; i < fdim; ++i) {
        freqs[i] = freq_min / std::pow(freq_base, static_cast<float>(i) / static_cast<float>(fdim));
    }
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const int32_t xyz[3] = {coords[r * 4 + 1], coords[r * 4 + 2], coords[r * 4 + 3]};
        const float * src = x + r * channels;
        float * dst = y + r * channels;
        for (int h = 0; h < heads; ++h) {
            for (int pr = 0; pr < pairs; ++pr) {
                float phase = 0.0f;
                if (pr < 3 * fdim) phase = static_cast<float>(xyz[pr / fdim]) * freqs[pr % fdim];
                const float cs = std::cos(phase);
                const float sn = std::sin(phase);
                const int off = h * head_dim + pr * 2;
                const float e = src[off];
                const float o = src[off + 1];
                dst[off] = e * cs - o * sn;
                dst[off + 1] = e * sn + o * cs;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// a7 / a9: attention for one query row against a contiguous key/value range,
// in the order of src/sparse.cpp:748-779 (and 823-855): scores = (q.k)*scale
// with the dot over dim ascending from 0; max; p = exp(s - max); denominator
// in key order; out += (p / denominator) * v in key order from 0.
static void attend_row(const float * q_row, const float * k_base, const float * v_base,
                       int64_t key_count, int heads, int head_dim, int v_head_dim,
                       int64_t k_stride, int64_t v_stride, float scale, float * out_row,
                       std::vector<float> & scores) {
    scores.resize(static_cast<size_t>(key_count));
    for (int h = 0; h < heads; ++h) {
        const float * qh = q_row + h * head_dim;
        float mx = -std::numeric_limits<float>::infinity();
        for (int64_t j = 0; j < key_count; ++j) {
            const float * kh = k_base + j * k_stride + h * head_dim;
            float s = 0.0f;
            for (int d = 0; d < head_dim; ++d) s += qh[d] * kh[d];
            scores[j] = s * scale;
            mx = std::max(mx, scores[j]);
        }
        float denom = 0.0f;
        for (int64_t j = 0; j < key_count; ++j) {
            scores[j] = std::exp(scores[j] - mx);
            denom += scores[j];
        }
        float * oh = out_row + h * v_head_dim;
        for (int d = 0; d < v_head_dim; ++d) oh[d] = 0.0f;
        for (int64_t j = 0; j < key_count; ++j) {
            const float prob = scores[j] / denom;
            const float * vh = v_base + j * v_stride + h * v_head_dim;
            for (int d = 0; d < v_head_dim; ++d) oh[d] += prob * vh[d];
        }
    }
}

// Varlen self-attention over segments: queries [cu_q[s], cu_q[s+1]) attend to
// keys/values [cu_k[s], cu_k[s+1]).  q,k: [*, heads*head_dim]; v: [*, heads*
// v_head_dim].  When rows is non-null only those query rows are computed
// (row sampling for the large configs); other output rows are untouched.
void orc_varlen_attention(const float * q, const float * k, const float * v, const int64_t * cu_q,
                          const int64_t * cu_k, int segments, int heads, int head_dim,
                          int v_head_dim, float scale, float * out, const int64_t * rows,
                          int64_t row_count) {
    const int64_t qc = static_cast<int64_t>(heads) * head_dim;
    const int64_t vc = static_cast<int64_t>(heads) * v_head_dim;
    std::vector<int64_t> all;
    if (!rows) {
        all.resize(static_cast<size_t>(cu_q[segments]));
        std::iota(all.begin(), all.end(), 0);
        rows = all.data();
        row_count = static_cast<int64_t>(all.size());
    }
#pragma omp parallel
    {
        std::vector<float> scores;
#pragma omp for schedule(dynamic, 16)
        for (int64_t i = 0; i < row_count; ++i) {
            const int64_t r = rows[i];
            int s = static_cast<int>(std::upper_bound(cu_q, cu_q + segments + 1, r) - cu_q) - 1;
            const int64_t kb = cu_k[s], ke = cu_k[s + 1];
            attend_row(q + r * qc, k + kb * qc, v + kb * vc, ke - kb, heads, head_dim, v_head_dim,
                       qc, vc, scale, out + r * vc, scores);
        }
    }
}

// cu_seqlens from a batch column: the reference scans for contiguous rows of
// equal batch (src/sparse.cpp:731-737).  cu has batch_size + 1 entries.
void orc_batch_cu_seqlens(const int32_t * coords, int64_t n, int batch_size, int64_t * cu) {
    int64_t p = 0;
    for (int b = 0; b < batch_size; ++b) {
        while (p < n && coords[p * 4] < b) ++p;
        cu[b] = p;
        while (p < n && coords[p * 4] == b) ++p;
    }
    cu[batch_size] = p;
}

// ---------------------------------------------------------------------------
// a8 (contract): shifted-window partition.  For each row, window
// (floor((x+s)/W), floor((y+s)/W), floor((z+s)/W)); per-axis window counts
// n_a = ceil((S_a + s)/W); wid = ((b*nx + wx)*ny + wy)*nz + wz.  fwd is the
// stable sort of rows by wid (fwd[i] = source row of permuted row i), bwd its
// inverse; cu_seqlens (length nwin + 1) bound the non-empty windows in
// ascending wid.  Returns nwin.
int64_t orc_window_partition(const int32_t * coords, int64_t n, int sx, int sy, int sz,
                             int window, int shift, int32_t * fwd, int32_t * bwd,
                             int64_t * cu_seqlens) {
    const int64_t nx = (sx + shift + window - 1) / window;
    const int64_t ny = (sy + shift + window - 1) / window;
    const int64_t nz = (sz + shift + window - 1) / window;
    std::vector<int64_t> wid(static_cast<size_t>(n));
    for (int64_t p = 0; p < n; ++p) {
        const int32_t * c = coords + p * 4;
        const int64_t wx = (c[1] + shift) / window;
        const int64_t wy = (c[2] + shift) / window;
        const int64_t wz = (c[3] + shift) / window;
        wid[p] = ((static_cast<int64_t>(c[0]) * nx + wx) * ny + wy) * nz + wz;
    }
    std::vector<int32_t> order(static_cast<size_t>(n));
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(),
                     [&](int32_t a, int32_t b) { return wid[a] < wid[b]; });
    int64_t nwin = 0;
    for (int64_t i = 0; i < n; ++i) {
        fwd[i] = order[i];
        bwd[order[i]] = static_cast<int32_t>(i);
        if (i == 0 || wid[order[i]] != wid[order[i - 1]]) cu_seqlens[nwin++] = i;
    }
    cu_seqlens[nwin] = n;
    return nwin;
}

// ---------------------------------------------------------------------------
// a13 helpers (src/sparse_transformer.cpp:71-121).
// modulate: y = x * (1 + (mod[off+C+c] + t[b][off+C+c])) + (mod[off+c] + t[b][off+c])
void orc_modulate(const int32_t * coords, const float * x, int64_t rows, int channels,
                  const float * block_mod, const float * t_mod, int offset, float * y) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const int b = coords[r * 4];
        const float * bm = t_mod + static_cast<int64_t>(b) * 6 * channels;
        for (int c = 0; c < channels; ++c) {
            const float scale = block_mod[offset + channels + c] + bm[offset + channels + c];
            const float shift = block_mod[offset + c] + bm[offset + c];
            y[r * channels + c] = x[r * channels + c] * (1.0f + scale) + shift;
        }
    }
}

// gate: x *= mod[off+c] + t[b][off+c]
void orc_gate(const int32_t * coords, float * x, int64_t rows, int channels,
              const float * block_mod, const float * t_mod, int offset) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const int b = coords[r * 4];
        const float * bm = t_mod + static_cast<int64_t>(b) * 6 * channels;
        for (int c = 0; c < channels; ++c) {
            x[r * channels + c] *= block_mod[offset + c] + bm[offset + c];
        }
    }
}

void orc_gelu_tanh(float * x, int64_t count) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) x[i] = gelu_tanh(x[i]);
}

void orc_silu(float * x, int64_t count) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) x[i] = silu_reciprocal_form(x[i]);
}

// ---------------------------------------------------------------------------
// a13: sparse_transformer_cross_block_f32 (src/sparse_transformer.cpp:138-292).
// w = the 23 block tensors in the order of SparseTransformerBlockWeightsF32.
// cfg_i = {channels, heads, mlp_hidden, context_channels, proj_in_channels,
// use_rope, qk_rms_norm, qk_rms_norm_cross, use_projection};
// cfg_f = {norm_eps, rope_freq_min, rope_freq_base}.  ctx_offsets has
// batch_size + 1 entries.  out may alias x.  rows, when non-null, restricts
// the block to sampled rows: the keys and values of the self-attention are
// computed for every row (each sampled query attends to all of its batch),
// every other linear and both attentions only for the sampled rows, and the
// row-local elementwise stages run over all rows.  Each sampled row of out
// then equals the full block's bit for bit; the other rows are meaningless.
void orc_transformer_block(const int32_t * coords, int64_t n, int batch_size, const float * x,
                           const float * t_mod, const float * ctx, const int64_t * ctx_offsets,
                           const float * projected, const int * cfg_i, const float * cfg_f,
                           const float * const * w, float * out, const int64_t * rows,
                           int64_t row_count) {
    const int C = cfg_i[0], H = cfg_i[1], M = cfg_i[2], CC = cfg_i[3], PC = cfg_i[4];
    const bool use_rope = cfg_i[5] != 0, qk_rms = cfg_i[6] != 0, qk_rms_cross = cfg_i[7] != 0;
    const bool use_proj = cfg_i[8] != 0;
    const float eps = cfg_f[0], fmin = cfg_f[1], fbase = cfg_f[2];
    const int D = C / H;
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    const float *mod = w[0], *qkv_w = w[1], *qkv_b = w[2], *q_g = w[3], *k_g = w[4];
    const float *out_w = w[5], *out_b = w[6], *n2_w = w[7], *n2_b = w[8];
    const float *cq_w = w[9], *cq_b = w[10], *ckv_w = w[11], *ckv_b = w[12];
    const float *cq_g = w[13], *ck_g = w[14], *co_w = w[15], *co_b = w[16];
    const float *pj_w = w[17], *pj_b = w[18], *m0_w = w[19], *m0_b = w[20];
    const float *m2_w = w[21], *m2_b = w[22];

    const size_t NC = static_cast<size_t>(n) * C;
    std::vector<float> h(x, x + NC);  // residual stream (alias-safe copy)
    std::vector<float> a(NC), b(NC);
    orc_layer_norm(h.data(), n, C, eps, nullptr, nullptr, a.data());
    orc_modulate(coords, a.data(), n, C, mod, t_mod, 0, b.data());
    // The fused QKV linear as its two halves: q (weight rows [0, C)) for the
    // query rows, k and v (weight rows [C, 3C)) for every row.
    std::vector<float> q(NC), k(NC), v(NC);
    linear_on_rows(b.data(), n, C, qkv_w, qkv_b, C, q.data(), rows, row_count);
    {
        std::vector<float> kv(static_cast<size_t>(n) * 2 * C);
        orc_linear(b.data(), n, C, qkv_w + static_cast<int64_t>(C) * C, qkv_b + C, 2 * C,
                   kv.data());
        for (int64_t r = 0; r < n; ++r) {
            std::memcpy(&k[r * C], &kv[r * 2 * C], sizeof(float) * C);
            std::memcpy(&v[r * C], &kv[r * 2 * C + C], sizeof(float) * C);
        }
    }
    if (qk_rms) {
        orc_mh_rms_norm(q.data(), n, H, D, q_g, a.data());
        q.swap(a);
        orc_mh_rms_norm(k.data(), n, H, D, k_g, a.data());
        k.swap(a);
    }
    if (use_rope) {
        orc_rope(coords, q.data(), n, H, D, fmin, fbase, a.data());
        q.swap(a);
        orc_rope(coords, k.data(), n, H, D, fmin, fbase, a.data());
        k.swap(a);
    }
    std::vector<int64_t> cu(static_cast<size_t>(batch_size) + 1);
    orc_batch_cu_seqlens(coords, n, batch_size, cu.data());
    std::vector<float> att(NC, 0.0f);
    orc_varlen_attention(q.data(), k.data(), v.data(), cu.data(), cu.data(), batch_size, H, D, D,
                         scale, att.data(), rows, row_count);
    linear_on_rows(att.data(), n, C, out_w, out_b, C, a.data(), rows, row_count);
    orc_gate(coords, a.data(), n, C, mod, t_mod, 2 * C);
    for (size_t i = 0; i < NC; ++i) h[i] += a[i];

    orc_layer_norm(h.data(), n, C, eps, n2_w, n2_b, b.data());
    std::vector<float> cq(NC);
    linear_on_rows(b.data(), n, C, cq_w, cq_b, C, cq.data(), rows, row_count);
    if (qk_rms_cross) {
        orc_mh_rms_norm(cq.data(), n, H, D, cq_g, a.data());
        cq.swap(a);
    }
    const int64_t T = ctx_offsets[batch_size];
    std::vector<float> ckv(static_cast<size_t>(T) * 2 * C);
    orc_linear(ctx, T, CC, ckv_w, ckv_b, 2 * C, ckv.data());
    std::vector<float> ck(static_cast<size_t>(T) * C), cv(static_cast<size_t>(T) * C);
    for (int64_t r = 0; r < T; ++r) {
        std::memcpy(&ck[r * C], &ckv[r * 2 * C], sizeof(float) * C);
        std::memcpy(&cv[r * C], &ckv[r * 2 * C + C], sizeof(float) * C);
    }
    if (qk_rms_cross) {
        std::vector<float> tmp(ck.size());
        orc_mh_rms_norm(ck.data(), T, H, D, ck_g, tmp.data());
        ck.swap(tmp);
    }
    std::fill(att.begin(), att.end(), 0.0f);
    orc_varlen_attention(cq.data(), ck.data(), cv.data(), cu.data(), ctx_offsets, batch_size, H,
                         D, D, scale, att.data(), rows, row_count);
    linear_on_rows(att.data(), n, C, co_w, co_b, C, a.data(), rows, row_count);
    if (use_proj) {
        linear_on_rows(projected, n, PC, pj_w, pj_b, C, b.data(), rows, row_count);
        for (size_t i = 0; i < NC; ++i) a[i] += b[i];
    }
    for (size_t i = 0; i < NC; ++i) h[i] += a[i];

    orc_layer_norm(h.data(), n, C, eps, nullptr, nullptr, a.data());
    orc_modulate(coords, a.data(), n, C, mod, t_mod, 3 * C, b.data());
    std::vector<float> hid(static_cast<size_t>(n) * M);
    linear_on_rows(b.data(), n, C, m0_w, m0_b, M, hid.data(), rows, row_count);
    orc_gelu_tanh(hid.data(), static_cast<int64_t>(hid.size()));
    linear_on_rows(hid.data(), n, M, m2_w, m2_b, C, a.data(), rows, row_count);
    orc_gate(coords, a.data(), n, C, mod, t_mod, 5 * C);
    for (size_t i = 0; i < NC; ++i) h[i] += a[i];
    std::memcpy(out, h.data(), NC * sizeof(float));
}

// ---------------------------------------------------------------------------
// a14: timestep embedding (src/flow.cpp:92-123) and MLP (src/flow.cpp:125-180).
void orc_timestep_embedding(const float * t, int64_t batch, int dim, int max_period, float * out) {
    const int half = dim / 2;
    const float log_period = static_cast<float>(std::log(static_cast<double>(max_period)));
    for (int64_t r = 0; r < batch; ++r) {
        float * dst = out + r * dim;
        for (int i = 0; i < half; ++i) {
            const float frac = static_cast<float>(i) / static_cast<float>(half);
            const float freq = std::exp(-log_period * frac);
            const float arg = t[r] * freq;
            dst[i] = std::cos(arg);
            dst[half + i] = std::sin(arg);
        }
        if (dim % 2 != 0) dst[dim - 1] = 0.0f;
    }
}

void orc_timestep_embed_mlp(const float * t, int64_t batch, int hidden, int freq_dim,
                            const float * w0, const float * b0, const float * w2,
                            const float * b2, float * out) {
    std::vector<float> f(static_cast<size_t>(batch) * freq_dim);
    orc_timestep_embedding(t, batch, freq_dim, 10000, f.data());
    std::vector<float> act(static_cast<size_t>(batch) * hidden);
    for (int64_t r = 0; r < batch; ++r) {
        for (int o = 0; o < hidden; ++o) {
            float acc = b0[o];
            for (int i = 0; i < freq_dim; ++i) acc += w0[static_cast<int64_t>(o) * freq_dim + i] * f[r * freq_dim + i];
            act[r * hidden + o] = silu_reciprocal_form(acc);
        }
    }
    for (int64_t r = 0; r < batch; ++r) {
        for (int o = 0; o < hidden; ++o) {
            float acc = b2[o];
            for (int i = 0; i < hidden; ++i) acc += w2[static_cast<int64_t>(o) * hidden + i] * act[r * hidden + i];
            out[r * hidden + o] = acc;
        }
    }
}

// a14: slat_flow_forward_f32 (src/slat_flow.cpp:161-249) in cross mode.
// fw = {input_w, input_b, t_w0, t_b0, t_w2, t_b2, mod_w, mod_b, out_w, out_b};
// blocks = num_blocks * 23 pointers.  dims = {in_ch, model_ch, out_ch,
// num_blocks, heads, mlp_hidden, cond_ch, qk_rms, qk_rms_cross};
// cfg_f = {norm_eps, rope_freq_min, rope_freq_base}.  rows: see
// orc_transformer_block.
void orc_slat_flow_forward(const int32_t * coords, int64_t n, int batch_size, const float * x,
                           const float * timesteps, const float * ctx, const int64_t * ctx_offsets,
                           const int * dims, const float * cfg_f, const float * const * fw,
                           const float * const * blocks, float * out, const int64_t * rows,
                           int64_t row_count) {
    const int IC = dims[0], C = dims[1], OC = dims[2], NB = dims[3];
    std::vector<float> h(static_cast<size_t>(n) * C);
    orc_linear(x, n, IC, fw[0], fw[1], C, h.data());
    std::vector<float> temb(static_cast<size_t>(batch_size) * C);
    orc_timestep_embed_mlp(timesteps, batch_size, C, 256, fw[2], fw[3], fw[4], fw[5], temb.data());
    for (float & value : temb) value = silu_branch_form(value);
    std::vector<float> tmod(static_cast<size_t>(batch_size) * 6 * C);
    orc_linear(temb.data(), batch_size, C, fw[6], fw[7], 6 * C, tmod.data());
    const int cfg_i[9] = {C, dims[4], dims[5], dims[6], 0, 1, dims[7], dims[8], 0};
    for (int blk = 0; blk < NB; ++blk) {
        orc_transformer_block(coords, n, batch_size, h.data(), tmod.data(), ctx, ctx_offsets,
                              nullptr, cfg_i, cfg_f, blocks + static_cast<int64_t>(blk) * 23,
                              h.data(), rows, row_count);
    }
    std::vector<float> normed(h.size());
    orc_layer_norm(h.data(), n, C, 1e-5f, nullptr, nullptr, normed.data());
    orc_linear(normed.data(), n, C, fw[8], fw[9], OC, out);
}

// ---------------------------------------------------------------------------
// a16: decoder blocks (src/slat_decoder.cpp:185-288).
// ConvNeXt: conv -> LN(affine) -> linear -> SiLU -> linear -> + input.
// w = {norm_w, norm_b, conv_w, conv_b, mlp0_w, mlp0_b, mlp2_w, mlp2_b}.
void orc_convnext_block(const int32_t * coords, int64_t n, const float * x, int channels,
                        int mlp_hidden, float eps, const float * const * w, float * out) {
    const size_t NC = static_cast<size_t>(n) * channels;
    std::vector<float> conv(NC), normed(NC), hid(static_cast<size_t>(n) * mlp_hidden), res(NC);
    orc_subm_conv3d(coords, n, x, channels, w[2], w[3], channels, conv.data());
    orc_layer_norm(conv.data(), n, channels, eps, w[0], w[1], normed.data());
    orc_linear(normed.data(), n, channels, w[4], w[5], mlp_hidden, hid.data());
    orc_silu(hid.data(), static_cast<int64_t>(hid.size()));
    orc_linear(hid.data(), n, mlp_hidden, w[6], w[7], channels, res.data());
    for (size_t i = 0; i < NC; ++i) res[i] += x[i];
    std::memcpy(out, res.data(), NC * sizeof(float));
}

// Channel-to-spatial residual block with a given subdivision (or none):
// LN(affine)+SiLU -> conv(C -> 8*out) -> C2S -> LN+SiLU -> conv(out -> out)
// + repeat(C2S(input)).  w = {norm1_w, norm1_b, conv1_w, conv1_b, conv2_w,
// conv2_b}.  Returns the output rows; out_coords holds 4*8n, out 8n*out_ch.
int64_t orc_resblock_c2s(const int32_t * coords, int64_t n, const float * x, int channels,
                         int out_channels, float eps, const float * subdivision,
                         const float * const * w, int32_t * out_coords, float * out) {
    const size_t NC = static_cast<size_t>(n) * channels;
    std::vector<float> normed(NC);
    orc_layer_norm(x, n, channels, eps, w[0], w[1], normed.data());
    orc_silu(normed.data(), static_cast<int64_t>(NC));
    const int packed_ch = out_channels * 8;
    std::vector<float> packed(static_cast<size_t>(n) * packed_ch);
    orc_subm_conv3d(coords, n, normed.data(), channels, w[2], w[3], packed_ch, packed.data());
    std::vector<int32_t> sc(static_cast<size_t>(n) * 32);
    std::vector<float> hidden(static_cast<size_t>(n) * packed_ch);
    const int64_t m = orc_channel_to_spatial(coords, n, packed.data(), packed_ch, 2, subdivision,
                                             sc.data(), hidden.data());
    std::vector<float> skip_sp(static_cast<size_t>(m) * (channels / 8));
    orc_channel_to_spatial(coords, n, x, channels, 2, subdivision, nullptr, skip_sp.data());
    const int skip_ch = channels / 8;
    const int repeats = out_channels / skip_ch;
    std::vector<float> hn(static_cast<size_t>(m) * out_channels);
    orc_layer_norm(hidden.data(), m, out_channels, eps, nullptr, nullptr, hn.data());
    orc_silu(hn.data(), static_cast<int64_t>(hn.size()));
    orc_subm_conv3d(sc.data(), m, hn.data(), out_channels, w[4], w[5], out_channels, out);
    for (int64_t r = 0; r < m; ++r) {
        // repeat_channels (src/slat_decoder.cpp:98-107): each source channel
        // repeated `repeats` times consecutively.
        for (int c = 0; c < skip_ch; ++c) {
            for (int rep = 0; rep < repeats; ++rep) {
                out[r * out_channels + c * repeats + rep] += skip_sp[r * skip_ch + c];
            }
        }
    }
    std::memcpy(out_coords, sc.data(), static_cast<size_t>(m) * 4 * sizeof(int32_t));
    return m;
}

// ---- flow Euler sampler (src/flow_sampler.cpp) -----------------------------

// Step schedule (src/flow_sampler.cpp:268-285) and configuration checks
// (111-124).  cfg = {sigma_min, rescale_t, guidance_strength, guidance_rescale,
// interval_min, interval_max}.  Returns 0, 1 (invalid configuration) or 2
// (non-finite schedule).
int orc_flow_schedule(int steps, const float * cfg, int step, float * t, float * t_next,
                      float * guidance) {
    const float sigma_min = cfg[0], rescale_t = cfg[1], strength = cfg[2], rescale = cfg[3];
    const float lo = cfg[4], hi = cfg[5];
    const bool bad = steps <= 0 || !(sigma_min >= 0.0f) || !(sigma_min < 1.0f) ||
                     !std::isfinite(sigma_min) || !(rescale_t > 0.0f) || !std::isfinite(rescale_t) ||
                     !std::isfinite(strength) || !std::isfinite(rescale) || rescale < 0.0f ||
                     !std::isfinite(lo) || !std::isfinite(hi) || lo > hi;
    if (bad) return 1;
    const float fsteps = static_cast<float>(steps);
    const float lin = 1.0f - static_cast<float>(step) / fsteps;
    const float den = 1.0f + (rescale_t - 1.0f) * lin;
    if (!(den > 0.0f) || !std::isfinite(den)) return 2;
    const float now = rescale_t * lin / den;
    const float lin_next = 1.0f - static_cast<float>(step + 1) / fsteps;
    const float den_next = 1.0f + (rescale_t - 1.0f) * lin_next;
    if (!(den_next > 0.0f) || !std::isfinite(den_next)) return 2;
    *t = now;
    *t_next = rescale_t * lin_next / den_next;
    *guidance = (now >= lo && now <= hi) ? strength : 1.0f;
    return 0;
}

// x0 = a * state - b * pred (src/flow_sampler.cpp:138-146).
static void flow_x0(const float * state, const float * pred, int64_t count, float t,
                    float sigma_min, float * x0) {
    const float a = 1.0f - sigma_min;
    const float b = sigma_min + a * t;
    for (int64_t i = 0; i < count; ++i) x0[i] = a * state[i] - b * pred[i];
}

// Population standard deviation per batch item, summed in row order
// (src/flow_sampler.cpp:158-190).  Returns false for an item without points.
static bool flow_batch_std(const int32_t * coords, const float * x, int64_t rows, int channels,
                           int batch, std::vector<float> & out) {
    std::vector<float> sum(batch, 0.0f), sum_sq(batch, 0.0f);
    std::vector<size_t> count(batch, 0);
    for (int64_t p = 0; p < rows; ++p) {
        const int b = coords[p * 4];
        for (int c = 0; c < channels; ++c) {
            const float v = x[p * channels + c];
            sum[b] += v;
            sum_sq[b] += v * v;
            ++count[b];
        }
    }
    out.assign(batch, 0.0f);
    for (int b = 0; b < batch; ++b) {
        if (count[b] == 0) return false;
        const float mean = sum[b] / static_cast<float>(count[b]);
        const float mean_sq = sum_sq[b] / static_cast<float>(count[b]);
        out[b] = std::sqrt(std::max(mean_sq - mean * mean, 0.0f));
    }
    return true;
}

// Guided prediction: the blend (src/flow_sampler.cpp:192-200), then the CFG
// rescale when rescale > 0 (202-235).  Returns 0, or 3 for an item without
// points.
int orc_flow_guidance(const float * state, const float * pos, const float * neg,
                      const int32_t * coords, int64_t rows, int channels, int batch, float t,
                      float sigma_min, float guidance, float rescale, float * pred) {
    const int64_t count = rows * channels;
    const float wn = 1.0f - guidance;
    for (int64_t i = 0; i < count; ++i) pred[i] = guidance * pos[i] + wn * neg[i];
    if (!(rescale > 0.0f)) return 0;
    std::vector<float> x0_pos(count), x0_cfg(count), sd_pos, sd_cfg;
    flow_x0(state, pos, count, t, sigma_min, x0_pos.data());
    flow_x0(state, pred, count, t, sigma_min, x0_cfg.data());
    if (!flow_batch_std(coords, x0_pos.data(), rows, channels, batch, sd_pos) ||
        !flow_batch_std(coords, x0_cfg.data(), rows, channels, batch, sd_cfg)) {
        return 3;
    }
    for (int64_t p = 0; p < rows; ++p) {
        const int b = coords[p * 4];
        const float ratio = sd_cfg[b] != 0.0f ? sd_pos[b] / sd_cfg[b] : 1.0f;
        for (int c = 0; c < channels; ++c) {
            float & v = x0_cfg[p * channels + c];
            const float scaled = v * ratio;
            v = rescale * scaled + (1.0f - rescale) * v;
        }
    }
    const float a = 1.0f - sigma_min;
    const float b = sigma_min + a * t;
    for (int64_t i = 0; i < count; ++i) pred[i] = (a * state[i] - x0_cfg[i]) / b;
    return 0;
}

// velocity(state, rows, channels, 1000 t, conditional, out, user): nonzero = ok.
typedef int (*orc_velocity_fn)(const float *, int64_t, int, float, int, float *, void *);

// flow_euler_sample_f32 (src/flow_sampler.cpp:237-345) without diagnostics.
// traj_xt / traj_x0 (nullable) receive steps x [rows, channels] each.
// Returns 0, the orc_flow_schedule / orc_flow_guidance codes, or 4 when the
// callback fails.
int orc_flow_euler_sample(const int32_t * coords, int64_t rows, int channels, int batch,
                          const float * noise, int steps, const float * cfg,
                          orc_velocity_fn model, void * user, float * samples, float * traj_xt,
                          float * traj_x0) {
    const int64_t count = rows * channels;
    float t0 = 0.0f, t1 = 0.0f, g0 = 0.0f;
    if (orc_flow_schedule(steps, cfg, 0, &t0, &t1, &g0) == 1) return 1;
    std::vector<float> state(noise, noise + count), pos(count), neg(count), pred(count);
    for (int step = 0; step < steps; ++step) {
        float t = 0.0f, t_next = 0.0f, g = 1.0f;
        if (int rc = orc_flow_schedule(steps, cfg, step, &t, &t_next, &g)) return rc;
        if (g == 1.0f || g == 0.0f) {
            if (!model(state.data(), rows, channels, 1000.0f * t, g == 1.0f ? 1 : 0, pred.data(),
                       user)) {
                return 4;
            }
        } else {
            if (!model(state.data(), rows, channels, 1000.0f * t, 1, pos.data(), user) ||
                !model(state.data(), rows, channels, 1000.0f * t, 0, neg.data(), user)) {
                return 4;
            }
            if (int rc = orc_flow_guidance(state.data(), pos.data(), neg.data(), coords, rows,
                                           channels, batch, t, cfg[0], g, cfg[3], pred.data())) {
                return rc;
            }
        }
        if (traj_x0) flow_x0(state.data(), pred.data(), count, t, cfg[0], traj_x0 + step * count);
        const float delta = t - t_next;
        for (int64_t i = 0; i < count; ++i) state[i] -= delta * pred[i];
        if (traj_xt) std::copy(state.begin(), state.end(), traj_xt + step * count);
    }
    std::copy(state.begin(), state.end(), samples);
    return 0;
}

int orc_thread_count() {
#if defined(_OPENMP)
    return omp_get_max_threads();
#else
    return 1;
#endif
}

} // extern "C"
