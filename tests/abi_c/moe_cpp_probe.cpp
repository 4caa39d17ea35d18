// A C++ caller of the MoE layer through include/exl3_moe.h only, the way an engine
// binds it: device buffers from hipMalloc, the linear descriptors, layer create,
// workspace query, one layer call on the default stream, destroy.
//
//   moe_cpp_probe layer.bin out.bin
//
// layer.bin (little-endian, written by tests/test_gpu_abi_cpp.py):
//   int32  H, I, E, top_k, n_group, topk_group, norm_topk_prob, shared (0 none, 1
//          trellis, 2 f16), SI, K_gu, cb_gu, K_dn, cb_dn, K_sh, cb_sh, B
//   float  routed_scaling_factor, swiglu_limit
//   per expert e, projection j (gate, up, down): trellis u16[(in/16)(out/16)16K],
//          suh u16[in], svh u16[out]
//   shared j = 0..2: trellis + suh + svh as above (K_sh, cb_sh), or f16 u16[in * out]
//   router u16[E * H], bias f32[E], h u16[B * H]
// out.bin: the layer output u16[B * H].
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "exl3_moe.h"

namespace {

FILE *g_in = nullptr;
std::vector<void *> g_dev;

void die(const char *what) {
  std::fprintf(stderr, "moe_cpp_probe: %s (%s)\n", what, exl3_last_error());
  std::exit(1);
}

template <typename T>
std::vector<T> read_n(size_t n) {
  std::vector<T> v(n);
  if (n && std::fread(v.data(), sizeof(T), n, g_in) != n) die("short layer file");
  return v;
}

template <typename T>
T *upload(const std::vector<T> &v) {
  void *p = nullptr;
  if (hipMalloc(&p, v.size() * sizeof(T) + 16) != hipSuccess) die("hipMalloc");
  if (hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) die("hipMemcpy");
  g_dev.push_back(p);
  return static_cast<T *>(p);
}

exl3_linear_desc trellis_linear(int in, int out, int K, int cb) {
  exl3_linear_desc d{};
  d.in_features = in;
  d.out_features = out;
  d.tw.trellis = upload(read_n<uint16_t>((size_t)(in / 16) * (out / 16) * 16 * K));
  d.tw.suh = upload(read_n<uint16_t>((size_t)in));
  d.tw.svh = upload(read_n<uint16_t>((size_t)out));
  d.tw.in_features = in;
  d.tw.out_features = out;
  d.tw.K = K;
  d.tw.codebook = cb;
  return d;
}

exl3_linear_desc dense_linear(int in, int out) {
  exl3_linear_desc d{};
  d.in_features = in;
  d.out_features = out;
  d.dense = upload(read_n<uint16_t>((size_t)in * out));
  return d;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: moe_cpp_probe layer.bin out.bin\n");
    return 2;
  }
  g_in = std::fopen(argv[1], "rb");
  if (!g_in) die("cannot open the layer file");
  const std::vector<int32_t> hd = read_n<int32_t>(16);
  const std::vector<float> hf = read_n<float>(2);
  const int H = hd[0], I = hd[1], E = hd[2], shared = hd[7], SI = hd[8], B = hd[15];
  std::vector<exl3_linear_desc> experts;
  for (int e = 0; e < E; ++e) {
    experts.push_back(trellis_linear(H, I, hd[9], hd[10]));
    experts.push_back(trellis_linear(H, I, hd[9], hd[10]));
    experts.push_back(trellis_linear(I, H, hd[11], hd[12]));
  }
  std::vector<exl3_linear_desc> sh;
  const int sdims[3][2] = {{H, SI}, {H, SI}, {SI, H}};
  for (int j = 0; shared && j < 3; ++j)
    sh.push_back(shared == 1 ? trellis_linear(sdims[j][0], sdims[j][1], hd[13], hd[14])
                             : dense_linear(sdims[j][0], sdims[j][1]));
  const uint16_t *router = upload(read_n<uint16_t>((size_t)E * H));
  const float *bias = upload(read_n<float>((size_t)E));
  const uint16_t *h = upload(read_n<uint16_t>((size_t)B * H));
  std::fclose(g_in);

  exl3_moe_layer_desc desc{experts.data(), sh.empty() ? nullptr : sh.data(), router, bias};
  exl3_moe_config cfg{H, I, E, hd[3], hd[4], hd[5], hd[6], hf[0], hf[1]};
  exl3_moe_layer_t layer = nullptr;
  if (exl3_moe_layer_create(&desc, &cfg, &layer) != EXL3_OK) die("exl3_moe_layer_create");
  const size_t ws_bytes = exl3_moe_workspace_size(layer, B);
  void *ws = nullptr;
  uint16_t *out = nullptr;
  if (hipMalloc(&ws, ws_bytes) != hipSuccess || hipMalloc((void **)&out, (size_t)B * H * 2) != hipSuccess)
    die("hipMalloc");
  if (exl3_moe_layer(layer, h, B, 1, out, ws, ws_bytes, nullptr) != EXL3_OK) die("exl3_moe_layer");
  if (hipDeviceSynchronize() != hipSuccess) die("hipDeviceSynchronize");
  std::vector<uint16_t> y((size_t)B * H);
  if (hipMemcpy(y.data(), out, y.size() * 2, hipMemcpyDeviceToHost) != hipSuccess) die("hipMemcpy");
  if (exl3_moe_layer_destroy(layer) != EXL3_OK) die("exl3_moe_layer_destroy");
  (void)hipFree(ws);
  (void)hipFree(out);
  for (void *p : g_dev) (void)hipFree(p);
  FILE *fo = std::fopen(argv[2], "wb");
  if (!fo || std::fwrite(y.data(), 2, y.size(), fo) != y.size()) die("cannot write the output");
  std::fclose(fo);
  std::printf("ok\n");
  return 0;
}
