// Host-side helpers shared by every entry point: error text, descriptor checks.
#include "rlm_common.hpp"

namespace rlm {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

const char* dtype_name(int d) {
  switch (d) {
    case RLM_F32: return "float32";
    case RLM_BF16: return "bfloat16";
    case RLM_F16: return "float16";
    case RLM_I32: return "int32";
    case RLM_I64: return "int64";
    default: return "unknown";
  }
}

bool check_tensor(const rlm_tensor* t, const char* name, int ndim) {
  if (t == nullptr) {
    set_error("%s: missing tensor", name);
    return false;
  }
  if (t->ndim != ndim) {
    set_error("%s: expected a %d-d tensor, got %d-d", name, ndim, t->ndim);
    return false;
  }
  int64_t numel = 1;
  for (int i = 0; i < ndim; ++i) {
    if (t->shape[i] < 0) {
      set_error("%s: negative size in dim %d", name, i);
      return false;
    }
    numel *= t->shape[i];
  }
  if (numel > 0 && t->data == nullptr) {
    set_error("%s: null data pointer", name);
    return false;
  }
  int64_t expected = 1;
  for (int i = ndim - 1; i >= 0; --i) {
    if (t->shape[i] != 1 && t->stride[i] != expected) {
      set_error("%s: must be contiguous (dim %d has stride %lld, expected %lld)", name, i,
                (long long)t->stride[i], (long long)expected);
      return false;
    }
    expected *= t->shape[i];
  }
  return true;
}

bool check_rows(const rlm_tensor* t, const char* name) {
  if (t == nullptr) {
    set_error("%s: missing tensor", name);
    return false;
  }
  if (t->ndim != 2) {
    set_error("%s: expected a 2-d tensor, got %d-d", name, t->ndim);
    return false;
  }
  if (t->shape[0] < 0 || t->shape[1] < 0) {
    set_error("%s: negative size", name);
    return false;
  }
  if (t->shape[0] * t->shape[1] > 0 && t->data == nullptr) {
    set_error("%s: null data pointer", name);
    return false;
  }
  if (t->shape[1] > 1 && t->stride[1] != 1) {
    set_error("%s: columns must be unit-stride (got stride %lld)", name, (long long)t->stride[1]);
    return false;
  }
  if (t->shape[0] > 1 && t->stride[0] < t->shape[1]) {
    set_error("%s: row stride %lld is smaller than the row width %lld", name,
              (long long)t->stride[0], (long long)t->shape[1]);
    return false;
  }
  return true;
}

bool check_dim(const rlm_tensor* t, const char* name, int dim, int64_t value) {
  if (t->shape[dim] != value) {
    set_error("%s: size %lld in dim %d does not match the expected %lld", name,
              (long long)t->shape[dim], dim, (long long)value);
    return false;
  }
  return true;
}

bool check_dtype_float(const rlm_tensor* t, const char* name) {
  if (!is_float_dtype(t->dtype)) {
    set_error("%s: expected float32/bfloat16/float16, got %s", name, dtype_name(t->dtype));
    return false;
  }
  return true;
}

bool check_dtype_is(const rlm_tensor* t, const char* name, int dtype) {
  if (t->dtype != dtype) {
    set_error("%s: expected %s, got %s", name, dtype_name(dtype), dtype_name(t->dtype));
    return false;
  }
  return true;
}

bool check_same_dtype(const rlm_tensor* a, const char* an, const rlm_tensor* b, const char* bn) {
  if (a->dtype != b->dtype) {
    set_error("%s (%s) and %s (%s) must share a dtype", an, dtype_name(a->dtype), bn,
              dtype_name(b->dtype));
    return false;
  }
  return true;
}

hipError_t launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return err;
}

}  // namespace rlm

extern "C" const char* rlm_last_error(void) { return rlm::g_last_error.c_str(); }

extern "C" const char* rlm_version(void) { return "relation_lm_hip 0.1.0 (gfx950)"; }
