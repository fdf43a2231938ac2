// op_check -- criterion program over the C++ operator layer.
//
// Links rpgbarenginecuda_amd/librpg_ops_objs.a (the objects of librpg_ops.so, C++
// symbols visible) and calls the operators through the reference's own C++
// signatures (namespace rpg; reference src/kernels_gpu.h:39-154), the way the
// engine's forward code would. The CPU oracle (oracle/cpu_ref.c) is linked as
// the checker. Every check prints its name before it launches anything.
//
//   [1] KV index map, integer-coded (values h*100 + t*10 + d, V = K + 1000) through
//       GpuKvWrite into GpuKvCache layer pointers; untouched slots stay zero;
//       an out-of-range write throws rpg::Error before launching
//   [2] GpuF16Sweep: all 65536 halves, bit-exact with the oracle
//   [3] GpuDequantRow and GpuEmbeddingLookup (GpuTensor) on synthetic Q4_K / Q6_K
//       rows, bit-exact with the oracle
//   [4] BuildRopeTable (host) bit-exact with the oracle's table; GpuRope matches
//       the oracle's RoPE bit for bit (same op order, no contraction)
//   [5] GpuAddRmsNorm: the residual add bit-exact
//
// Exit status: 0 all checks passed, 1 a check failed, 2 no usable device.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../oracle/cpu_ref.h"
#include "kernels_gpu.h"

namespace {

int g_fail = 0;

void Check(bool ok, const char* what) {
  std::printf("  [%s] %s\n", ok ? " OK " : "FAIL", what);
  std::fflush(stdout);
  if (!ok) ++g_fail;
}

void Case(const char* name) {
  std::printf("[case] %s\n", name);
  std::fflush(stdout);
}

uint64_t g_rng = 0x5EED2026ull;
uint32_t NextU32() {
  uint64_t z = (g_rng += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return static_cast<uint32_t>((z ^ (z >> 31)) >> 16);
}

float NextF(float lo, float hi) { return lo + (hi - lo) * static_cast<float>(NextU32() & 0xFFFFFF) / 16777216.0f; }

template <typename T>
void Up(rpg::DeviceBuffer& d, const std::vector<T>& h) {
  d.Alloc(h.size() * sizeof(T));
  d.Upload(h.data(), h.size() * sizeof(T));
}

template <typename T>
std::vector<T> Down(const rpg::DeviceBuffer& d, size_t n) {
  std::vector<T> h(n);
  RPG_HIP_CHECK(hipDeviceSynchronize());
  d.Download(h.data(), n * sizeof(T));
  return h;
}

// Synthetic quant rows: random bytes, with the fp16 scales set to small finite values.
std::vector<uint8_t> QuantRows(uint32_t type, int64_t rows, int64_t cols) {
  const int64_t nb = cols / 256;
  const int64_t bb = type == rpg::kGgmlQ4_K ? 144 : 210;
  std::vector<uint8_t> t(static_cast<size_t>(rows * nb * bb));
  for (auto& b : t) b = static_cast<uint8_t>(NextU32());
  for (int64_t blk = 0; blk < rows * nb; ++blk) {
    uint8_t* p = t.data() + blk * bb;
    const uint16_t d = ora_f32_to_f16_rne(NextF(0.0f, 0.02f));
    const uint16_t m = ora_f32_to_f16_rne(NextF(0.0f, 0.02f));
    if (type == rpg::kGgmlQ4_K) {
      std::memcpy(p, &d, 2);
      std::memcpy(p + 2, &m, 2);
    } else {
      std::memcpy(p + 208, &d, 2);
    }
  }
  return t;
}

bool SameBits(const float* a, const float* b, size_t n) { return std::memcmp(a, b, n * sizeof(float)) == 0; }

void KvMapCheck() {
  Case("[1] KV index map via GpuKvCache + GpuKvWrite");
  rpg::ModelMeta c;
  c.n_layers = 2;
  c.n_kv_heads = 3;
  c.head_dim = 8;
  const int64_t max_seq = 12, pos0 = 4, seq = 5;
  rpg::GpuKvCache cache(c, max_seq);
  const size_t layer_elems = static_cast<size_t>(c.n_kv_heads * max_seq * c.head_dim);
  RPG_HIP_CHECK(hipMemset(cache.k_layer(0), 0, 2 * layer_elems * 2));  // both layers of K
  RPG_HIP_CHECK(hipMemset(cache.v_layer(0), 0, 2 * layer_elems * 2));
  std::vector<float> k(static_cast<size_t>(seq * c.n_kv_heads * c.head_dim)), v(k.size());
  for (int64_t t = 0; t < seq; ++t)
    for (int h = 0; h < c.n_kv_heads; ++h)
      for (int d = 0; d < c.head_dim; ++d) {
        const size_t i = static_cast<size_t>((t * c.n_kv_heads + h) * c.head_dim + d);
        k[i] = static_cast<float>(h * 100 + t * 10 + d);
        v[i] = k[i] + 1000.0f;
      }
  rpg::DeviceBuffer kd, vd;
  Up(kd, k);
  Up(vd, v);
  rpg::GpuKvWrite(static_cast<const float*>(kd.data()), static_cast<const float*>(vd.data()), c.n_kv_heads,
                  c.head_dim, pos0, seq, cache.k_layer(1), cache.v_layer(1), max_seq);
  std::vector<uint16_t> kh(2 * layer_elems), vh(2 * layer_elems);
  RPG_HIP_CHECK(hipDeviceSynchronize());
  RPG_HIP_CHECK(hipMemcpy(kh.data(), cache.k_layer(0), kh.size() * 2, hipMemcpyDeviceToHost));
  RPG_HIP_CHECK(hipMemcpy(vh.data(), cache.v_layer(0), vh.size() * 2, hipMemcpyDeviceToHost));
  int64_t bad = 0, dirty = 0;
  for (int layer = 0; layer < 2; ++layer)
    for (int h = 0; h < c.n_kv_heads; ++h)
      for (int64_t p = 0; p < max_seq; ++p)
        for (int d = 0; d < c.head_dim; ++d) {
          const size_t o = layer * layer_elems + static_cast<size_t>((h * max_seq + p) * c.head_dim + d);
          const bool written = layer == 1 && p >= pos0 && p < pos0 + seq;
          if (!written) {
            dirty += (kh[o] != 0) + (vh[o] != 0);
            continue;
          }
          const float want = static_cast<float>(h * 100 + (p - pos0) * 10 + d);
          bad += ora_f16_to_f32(kh[o]) != want;
          bad += ora_f16_to_f32(vh[o]) != want + 1000.0f;
        }
  Check(bad == 0, "120 written K/V elements equal their integer codes, bit-exact");
  Check(dirty == 0, "every other slot of both layers stays zero");
  bool threw = false;
  try {
    rpg::GpuKvWrite(static_cast<const float*>(kd.data()), static_cast<const float*>(vd.data()), c.n_kv_heads,
                    c.head_dim, 8, seq, cache.k_layer(1), cache.v_layer(1), max_seq);
  } catch (const rpg::Error&) {
    threw = true;
  }
  Check(threw, "a write past max_seq throws rpg::Error before launching");
}

void F16Sweep() {
  Case("[2] GpuF16Sweep, all 65536 halves");
  rpg::DeviceBuffer out(65536 * sizeof(float));
  rpg::GpuF16Sweep(static_cast<float*>(out.data()));
  const std::vector<float> got = Down<float>(out, 65536);
  std::vector<uint16_t> bits(65536);
  for (int i = 0; i < 65536; ++i) bits[static_cast<size_t>(i)] = static_cast<uint16_t>(i);
  std::vector<float> want(65536);
  ora_f16_to_f32_array(bits.data(), 65536, want.data());
  Check(SameBits(got.data(), want.data(), 65536), "device f16 -> f32 equals the oracle on every pattern");
}

void DequantAndGather() {
  for (uint32_t type : {rpg::kGgmlQ4_K, rpg::kGgmlQ6_K}) {
    Case(type == rpg::kGgmlQ4_K ? "[3] Q4_K dequant row + GpuEmbeddingLookup"
                                : "[3] Q6_K dequant row + GpuEmbeddingLookup");
    const int64_t rows = 97, cols = 2048;
    const std::vector<uint8_t> table = QuantRows(type, rows, cols);
    rpg::GpuTensor emb;
    Up(emb.buf, table);
    emb.type = type;
    emb.matrix = true;
    emb.rows = rows;
    emb.cols = cols;
    emb.n_elements = rows * cols;
    const int64_t rb = emb.row_bytes();

    rpg::DeviceBuffer row_out(cols * sizeof(float));
    rpg::GpuDequantRow(type, static_cast<const uint8_t*>(emb.buf.data()) + 5 * rb, cols,
                       static_cast<float*>(row_out.data()));
    std::vector<float> want(static_cast<size_t>(cols));
    ora_dequantize_row(type, table.data() + 5 * rb, cols, want.data());
    Check(SameBits(Down<float>(row_out, cols).data(), want.data(), cols), "GpuDequantRow is bit-exact");

    const std::vector<int32_t> toks = {0, 96, 5, 5, 41, 17, 96};
    rpg::DeviceBuffer tok_dev, x(toks.size() * cols * sizeof(float));
    Up(tok_dev, toks);
    rpg::GpuEmbeddingLookup(emb, static_cast<const int32_t*>(tok_dev.data()), static_cast<int64_t>(toks.size()),
                            static_cast<float*>(x.data()));
    std::vector<float> gwant(toks.size() * cols);
    ora_embedding_lookup(type, table.data(), rows, cols, toks.data(), static_cast<int64_t>(toks.size()), gwant.data());
    Check(SameBits(Down<float>(x, gwant.size()).data(), gwant.data(), gwant.size()),
          "GpuEmbeddingLookup(GpuTensor) is bit-exact");
  }
}

void RopeTableAndRope() {
  Case("[4] BuildRopeTable + GpuRope");
  const int32_t d = 128, heads = 8;
  const int64_t n_pos = 4096, rows = 33, pos0 = 1000;
  const std::vector<float> tab = rpg::BuildRopeTable(d, 1e6, n_pos);
  std::vector<float> want_tab(tab.size());
  ora_build_rope_table(d, 1e6, n_pos, want_tab.data());
  Check(SameBits(tab.data(), want_tab.data(), tab.size()), "host RoPE table equals the oracle's, bit for bit");
  std::vector<float> x(static_cast<size_t>(rows * heads * d));
  for (auto& e : x) e = NextF(-2.0f, 2.0f);
  rpg::DeviceBuffer xd, td;
  Up(xd, x);
  Up(td, tab);
  rpg::GpuRope(static_cast<float*>(xd.data()), heads, d, static_cast<const float*>(td.data()), pos0, rows);
  std::vector<float> want = x;
  ora_rope(want.data(), heads, d, tab.data(), pos0, rows);
  Check(SameBits(Down<float>(xd, x.size()).data(), want.data(), x.size()), "GpuRope equals the oracle bit for bit");
}

void AddRmsNorm() {
  Case("[5] GpuAddRmsNorm residual add");
  const int64_t rows = 21, n = 2048;
  std::vector<float> x(static_cast<size_t>(rows * n)), dl(x.size()), w(static_cast<size_t>(n));
  for (auto& e : x) e = NextF(-3.0f, 3.0f);
  for (auto& e : dl) e = NextF(-3.0f, 3.0f);
  for (auto& e : w) e = NextF(0.8f, 1.2f);
  rpg::DeviceBuffer xd, dd, wd, hd(x.size() * sizeof(float));
  Up(xd, x);
  Up(dd, dl);
  Up(wd, w);
  rpg::GpuAddRmsNorm(static_cast<float*>(xd.data()), static_cast<const float*>(dd.data()),
                     static_cast<const float*>(wd.data()), rows, n, 1e-6f, static_cast<float*>(hd.data()));
  std::vector<float> sum = x;
  ora_vec_add(sum.data(), dl.data(), static_cast<int64_t>(sum.size()));
  Check(SameBits(Down<float>(xd, x.size()).data(), sum.data(), sum.size()), "x + d is bit-exact");
}

}  // namespace

int main() {
  const rpg::DeviceInfo dev = rpg::QueryDevice(0);
  std::printf("%s\n", rpg::DescribeDevice(dev).c_str());
  if (!dev.available) return 2;
  try {
    KvMapCheck();
    F16Sweep();
    DequantAndGather();
    RopeTableAndRope();
    AddRmsNorm();
  } catch (const std::exception& e) {
    std::printf("error: %s\n", e.what());
    return 1;
  }
  std::printf("%s\n", g_fail == 0 ? "PASS" : "FAIL");
  return g_fail == 0 ? 0 : 1;
}
