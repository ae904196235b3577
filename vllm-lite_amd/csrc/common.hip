// Error reporting and device queries shared by all entry points.
#include <stdarg.h>
#include <stdio.h>

#include "vl_common.h"

static thread_local char g_err[512] = "";

void vl_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

extern "C" const char* vl_last_error(void) { return g_err; }

extern "C" int vl_abi_version(void) { return 13; }

int vl_num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

int vl_kv_geom(int kv_layout, int block_size, int num_kv_heads, int head_dim, KvGeom* g) {
  VL_CHECK_ARG(num_kv_heads > 0 && head_dim > 0, "bad shape");
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (kv_layout == VL_KV_TOKEN_MAJOR) {
    *g = KvGeom{row, row, head_dim, 0};
    return VL_OK;
  }
  VL_CHECK_ARG(kv_layout == VL_KV_HEAD_MAJOR, "bad kv_layout %d", kv_layout);
  VL_CHECK_ARG(block_size > 0 && (block_size & (block_size - 1)) == 0,
               "head-major caches need a power-of-two block_size (got %d)", block_size);
  int lg = 0;
  while ((1 << lg) < block_size) ++lg;
  *g = KvGeom{row << lg, head_dim, (int64_t)head_dim << lg, lg};
  return VL_OK;
}
