// A C++ host driver of the model-level boundary, in place of
// src/main_big.cpp:332-369 (main): layout -> blob -> q3_model_open ->
// q3_generate -> copy the blob back and read its ids and logits.  The model is config 0's random-init blob (one layer,
// 1024-token vocab, a 40-token prompt as 32 + 8 rows, 2 greedy tokens) in
// mode 1, so the last forward's logits are written.  Usage:
//   generate_cfg0 OUT.bin   -> OUT.bin holds int32 ids[40..41] then the f32
//                              logits row; exit status 0 on success.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <vector>

#include "q3ops.h"

static int fail(const char *what, int rc) {
  std::fprintf(stderr, "%s failed: %d\n", what, rc);
  return 1;
}

int main(int argc, char **argv) {
  if (argc != 2) return fail("usage: generate_cfg0 OUT.bin", 2);
  q3_layout lay;
  int rc = q3_layout_compute(1024, 1, 16, 8, 128, 3072, 1024, /*seq*/ 32, /*max_seq*/ 256, &lay);
  if (rc != Q3_OK) return fail("q3_layout_compute", rc);
  // the blob the reference's tools write (here: the random-init stand-in)
  q3_init_params p{};
  p.weight_seed = 0x5EED0000ull;
  p.ids_seed = 0x5EED0001ull;
  p.weight_std = 0.02;
  p.gain_std = 0.05;
  p.rope_theta = 1e6;
  p.n_prompt = 40;
  p.n_gen = 2;
  p.mode = 1;  // full logits of the last forward
  std::vector<uint8_t> host(static_cast<size_t>(lay.kSCRATCH_END));
  rc = q3_init_random_blob(&lay, &p, host.data(), 0);
  if (rc != Q3_OK) return fail("q3_init_random_blob", rc);
  void *blob = nullptr;
  if (hipMalloc(&blob, host.size()) != hipSuccess) return fail("hipMalloc", -1);
  if (hipMemcpy(blob, host.data(), host.size(), hipMemcpyHostToDevice) != hipSuccess) return fail("hipMemcpy", -1);
  q3_model *m = nullptr;
  rc = q3_model_open(blob, &lay, nullptr, &m);
  if (rc != Q3_OK) return fail("q3_model_open", rc);
  rc = q3_generate(m);  // CTRL -> chunked prefill -> greedy decode -> ids[]
  if (rc != Q3_OK) return fail("q3_generate", rc);
  if (hipDeviceSynchronize() != hipSuccess) return fail("hipDeviceSynchronize", -1);
  if (hipMemcpy(host.data(), blob, host.size(), hipMemcpyDeviceToHost) != hipSuccess) return fail("hipMemcpy", -1);
  rc = q3_model_close(m);
  if (rc != Q3_OK) return fail("q3_model_close", rc);
  (void)hipFree(blob);
  std::FILE *f = std::fopen(argv[1], "wb");
  if (!f) return fail("fopen", -1);
  const int32_t *ids = reinterpret_cast<const int32_t *>(host.data() + lay.kIDS);
  const float *logits = reinterpret_cast<const float *>(host.data() + lay.kLOGITS);
  const bool ok = std::fwrite(ids + 40, sizeof(int32_t), 2, f) == 2 &&
                  std::fwrite(logits, sizeof(float), lay.vocab, f) == lay.vocab;
  std::fclose(f);
  if (!ok) return fail("fwrite", -1);
  std::printf("ids %d %d\n", ids[40], ids[41]);
  return 0;
}
