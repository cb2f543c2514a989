// Host-only driver for the GGUF reader under AddressSanitizer (tests only):
// opens every file named on the command line with pbx_gguf_open and, when
// that succeeds, walks the tensor table, the metadata accessors and the
// model-config extraction.  The model and runtime entry points the reader's
// loader refers to are stubbed; the loader itself is not called.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "pbx_internal.h"

static std::string g_msg;
int pbx_fail(pbx_ctx *, int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_msg = buf;
  return code;
}
extern "C" const char *pbx_last_error(const pbx_ctx *) { return g_msg.c_str(); }
size_t pbx_type_row_bytes(int, int64_t) { return 0; }
extern "C" int pbx_model_create(pbx_ctx *, const pbx_model_config *, pbx_model **) { return -1; }
extern "C" int pbx_model_set_tensor(pbx_model *, int, int, const void *, size_t) { return -1; }
extern "C" int pbx_model_free(pbx_model *) { return 0; }

int main(int argc, char **argv) {
  int opened = 0;
  for (int a = 1; a < argc; ++a) {
    pbx_gguf *g = nullptr;
    if (pbx_gguf_open(argv[a], &g) != PBX_OK) continue;
    ++opened;
    int64_t nt = 0, nk = 0;
    uint32_t ver;
    uint64_t ds;
    pbx_gguf_info(g, &ver, &nt, &nk, &ds);
    unsigned sum = 0;
    for (int64_t i = 0; i < nt; ++i) {
      pbx_gguf_tensor t;
      if (pbx_gguf_tensor_info(g, i, &t) != PBX_OK) return 2;
      const unsigned char *p = (const unsigned char *)t.data;
      for (uint64_t k = 0; k < t.nbytes; k += 61) sum += p[k];  // touch the data
      if (t.nbytes) sum += p[t.nbytes - 1];
      if (pbx_gguf_find_tensor(g, t.name) < 0) return 3;
    }
    int64_t iv;
    double fv;
    const char *s;
    uint64_t n;
    uint32_t et;
    const char *keys[] = {"general.architecture", "general.alignment", "llama.block_count",
                          "tokenizer.ggml.tokens", "v.str", "v.arr_str", "v.f64"};
    for (const char *k : keys) {
      pbx_gguf_get_int(g, k, &iv);
      pbx_gguf_get_float(g, k, &fv);
      if (pbx_gguf_get_string(g, k, &s, &n) == PBX_OK && n) sum += (unsigned char)s[n - 1];
      pbx_gguf_get_array(g, k, &et, &n);
    }
    pbx_model_config cfg;
    pbx_gguf_model_config(g, 0, &cfg);
    pbx_gguf_close(g);
    if (sum == 0xFFFFFFFFu) printf(".");
  }
  printf("opened %d of %d\n", opened, argc - 1);
  return 0;
}
