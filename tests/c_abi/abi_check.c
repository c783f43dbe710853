/* A C99 caller of include/q3ops.h (no GPU needed): the blob layout of the
 * default Qwen3-0.6B shape and of config 0, the model_big.h header text and
 * the host-side error paths.  Prints one "key value" line per result; the
 * test that builds this file (tests/test_c_abi.py) compares them. */
#include <stdio.h>
#include <string.h>

#include "q3ops.h"

int main(void) {
  q3_layout lay, small;
  q3_model *m = NULL;
  char hdr[64];
  int rc;
  float w[2 * 4] = {0.5f, -1.0f, 0.25f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  int8_t q[2 * 4];
  float s[2];

  /* tools/pqwf.py Layout at the default shape (main_big.cpp's model) */
  rc = q3_layout_compute(1024, 28, 16, 8, 128, 3072, 151936, 32, 256, &lay);
  printf("layout_rc %d\n", rc);
  printf("kSCRATCH_END %lld\n", (long long)lay.kSCRATCH_END);
  printf("kKV_STRIDE %lld\n", (long long)lay.kKV_STRIDE);
  printf("kKV_VOFF %lld\n", (long long)lay.kKV_VOFF);
  printf("kLOGITS %lld\n", (long long)lay.kLOGITS);
  /* config 0: one layer, 1024-token vocab */
  rc = q3_layout_compute(1024, 1, 16, 8, 128, 3072, 1024, 32, 256, &small);
  printf("cfg0_rc %d\n", rc);
  printf("cfg0_kSCRATCH_END %lld\n", (long long)small.kSCRATCH_END);
  /* header text: the length needed, NUL-terminated within a short buffer */
  rc = q3_layout_header_text(&lay, hdr, sizeof hdr);
  printf("header_len %d\n", rc);
  printf("header_nul %d\n", (int)(memchr(hdr, 0, sizeof hdr) != NULL));
  /* host error paths: no GPU is touched */
  printf("layout_null %d\n", q3_layout_compute(1024, 28, 16, 8, 128, 3072, 151936, 32, 256, NULL));
  printf("open_null %d\n", q3_model_open(NULL, &lay, NULL, &m));
  printf("open_null_layout %d\n", q3_model_open(hdr, NULL, NULL, &m));
  printf("generate_null %d\n", q3_generate(NULL));
  printf("close_null %d\n", q3_model_close(NULL));
  /* tools/pqwf.py:72-89 quantize_rows: scale = max|w| / 127, q = rint(w / scale) */
  rc = q3_quantize_rows_host(w, 2, 4, q, s);
  printf("quant_rc %d\n", rc);
  printf("quant_row0 %d %d %d %d\n", q[0], q[1], q[2], q[3]);
  printf("quant_row1_zero %d\n", (int)(q[4] == 0 && q[5] == 0 && s[1] == 0.0f));
  printf("Q3_OK %d Q3_ERR_ARG %d\n", Q3_OK, Q3_ERR_ARG);
  return 0;
}
