/* bundle.h — reader of the model bundles tests/native/bundle.py writes (a synthetic GGUF's
 * tensors, the oracle and library model configs, KV capacities and a prompt). Shared by the
 * sanitizer drivers; every field is bounds-checked against the file size. */
#ifndef WGD_BUNDLE_H
#define WGD_BUNDLE_H
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  char name[128];
  int32_t type;
  uint32_t n_dims;
  uint64_t dims[4];
  uint64_t bytes;
  const uint8_t *data;
} bundle_tensor;

typedef struct {
  uint8_t *file;
  uint64_t size, at;
  const uint8_t *orc_cfg, *wgd_cfg;
  uint32_t orc_cfg_size, wgd_cfg_size;
  uint32_t layers, n_prompt, chunk, steps, n_tensors;
  int32_t *capacities, *prompt;
  bundle_tensor *tensors;
} bundle;

static int bundle_take(bundle *b, void *dst, uint64_t n) {
  if (n > b->size - b->at) return 1;
  if (dst) memcpy(dst, b->file + b->at, (size_t)n);
  b->at += n;
  return 0;
}

static void bundle_free(bundle *b) {
  free(b->file); free(b->capacities); free(b->prompt); free(b->tensors);
  memset(b, 0, sizeof(*b));
}

/* 0 on success; the bundle owns its buffers until bundle_free. */
static int bundle_read(const char *path, bundle *b) {
  memset(b, 0, sizeof(*b));
  FILE *fh = fopen(path, "rb");
  if (!fh) return 1;
  if (fseek(fh, 0, SEEK_END) || (long)(b->size = (uint64_t)ftell(fh)) < 0 || fseek(fh, 0, SEEK_SET)) { fclose(fh); return 1; }
  b->file = (uint8_t *)malloc(b->size ? (size_t)b->size : 1);
  if (!b->file || fread(b->file, 1, (size_t)b->size, fh) != b->size) { fclose(fh); bundle_free(b); return 1; }
  fclose(fh);
  char magic[4]; uint32_t version;
  if (bundle_take(b, magic, 4) || memcmp(magic, "WGDB", 4) || bundle_take(b, &version, 4) || version != 1) goto bad;
  if (bundle_take(b, &b->orc_cfg_size, 4)) goto bad;
  b->orc_cfg = b->file + b->at;
  if (bundle_take(b, NULL, b->orc_cfg_size) || bundle_take(b, &b->wgd_cfg_size, 4)) goto bad;
  b->wgd_cfg = b->file + b->at;
  if (bundle_take(b, NULL, b->wgd_cfg_size) || bundle_take(b, &b->layers, 4) || b->layers > 4096) goto bad;
  b->capacities = (int32_t *)calloc(b->layers + 1, 4);
  if (!b->capacities || bundle_take(b, b->capacities, 4ull * b->layers)) goto bad;
  if (bundle_take(b, &b->n_prompt, 4) || b->n_prompt > (1u << 20)) goto bad;
  b->prompt = (int32_t *)calloc(b->n_prompt + 1, 4);
  if (!b->prompt || bundle_take(b, b->prompt, 4ull * b->n_prompt)) goto bad;
  if (bundle_take(b, &b->chunk, 4) || bundle_take(b, &b->steps, 4) || !b->chunk) goto bad;
  if (bundle_take(b, &b->n_tensors, 4) || b->n_tensors > (1u << 16)) goto bad;
  b->tensors = (bundle_tensor *)calloc(b->n_tensors + 1, sizeof(bundle_tensor));
  if (!b->tensors) goto bad;
  for (uint32_t i = 0; i < b->n_tensors; i++) {
    bundle_tensor *t = &b->tensors[i];
    uint32_t len;
    if (bundle_take(b, &len, 4) || len >= sizeof(t->name) || bundle_take(b, t->name, len)) goto bad;
    t->name[len] = 0;
    if (bundle_take(b, &t->type, 4) || bundle_take(b, &t->n_dims, 4) || t->n_dims < 1 || t->n_dims > 4) goto bad;
    if (bundle_take(b, t->dims, 8ull * t->n_dims) || bundle_take(b, &t->bytes, 8)) goto bad;
    t->data = b->file + b->at;
    if (bundle_take(b, NULL, t->bytes)) goto bad;
  }
  if (b->at != b->size) goto bad;
  return 0;
bad:
  bundle_free(b);
  return 2;
}

static int bundle_write(const char *path, const void *data, uint64_t bytes, const char *mode) {
  FILE *fh = fopen(path, mode);
  if (!fh) return 1;
  int rc = fwrite(data, 1, (size_t)bytes, fh) != bytes;
  return fclose(fh) || rc;
}
#endif
