// N-API addon: the Node side of the sampler's C ABI (include/tabby_sampler.h).
//
// It stays thin on purpose. Argument checking, the reference's error messages, the RNG
// and the SampleOutcome objects live in index.js; this file only moves bytes:
//   create / destroy             tabby_sampler_create / _destroy (ForwardPass scratch,
//                                src/engine/forward.ts:243-248, 309-315)
//   deviceAlloc / deviceFree /   device buffers for logits that the host holds (the
//   upload                       reference's logits are already on its GPU; here a caller
//                                without a HIP producer uploads them once)
//   wrapDevicePointer            logits a HIP producer in this process already wrote
//   sample                       tabby_sampler_sample: params packed by index.js as
//                                tabby_row_params, results returned as tabby_row_result bytes
//                                (encodeSampling + readback, forward.ts:442-451, 522-601)
//   argmax                       tabby_argmax_device + a 4-byte-per-row readback (the greedy
//                                path: sampler.ts:13-23, inference.worker.ts:216-229)
//   softmaxRows / download       tabby_softmax_rows_device between device buffers, and a
//                                device -> host copy (softmax_rows.wgsl, forward.ts:912-926)
//   version
#define NAPI_VERSION 6
#include <node_api.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>

#include "tabby_sampler.h"

namespace {

struct Handle {
  tabby_sampler *sampler = nullptr;
  int device = 0;
  int32_t *ids_dev = nullptr;  // argmax results, grown to the largest batch seen
  size_t ids_cap = 0;
};

struct DeviceBuffer {
  void *ptr = nullptr;
  size_t bytes = 0;
  int device = 0;
  bool owned = true;  // false for a caller's pointer (wrapDevicePointer): never freed here
};

napi_value fail(napi_env env, const std::string &msg) {
  napi_throw_error(env, nullptr, msg.c_str());
  return nullptr;
}

#define CHECK_NAPI(env, call)                                        \
  do {                                                               \
    if ((call) != napi_ok) return fail((env), "N-API call failed: " #call); \
  } while (0)

bool get_args(napi_env env, napi_callback_info info, size_t want, napi_value *argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok) return false;
  return argc == want;
}

bool get_i64(napi_env env, napi_value v, int64_t *out) {
  return napi_get_value_int64(env, v, out) == napi_ok;
}

// An argument the C ABI takes as int32_t: in [lo, INT32_MAX].
bool in_i32(int64_t v, int64_t lo) { return v >= lo && v <= INT32_MAX; }

// rows x cols entries of `elem` bytes fit in `cap` bytes, with both counts in [1, INT32_MAX]
// (the C ABI's int32_t); checked by division, so no product can overflow.
bool dims_fit(int64_t rows, int64_t cols, size_t elem, size_t cap) {
  if (!in_i32(rows, 1) || !in_i32(cols, 1)) return false;
  return (uint64_t)rows <= cap / elem / (uint64_t)cols;
}

void release_handle(Handle *h) {
  if (h->sampler) tabby_sampler_destroy(h->sampler);
  h->sampler = nullptr;
  if (h->ids_dev) {
    (void)hipSetDevice(h->device);
    (void)hipFree(h->ids_dev);
  }
  h->ids_dev = nullptr;
  h->ids_cap = 0;
}

void finalize_handle(napi_env, void *data, void *) {
  Handle *h = static_cast<Handle *>(data);
  release_handle(h);
  delete h;
}

void finalize_buffer(napi_env, void *data, void *) {
  DeviceBuffer *b = static_cast<DeviceBuffer *>(data);
  if (b->ptr && b->owned) {
    (void)hipSetDevice(b->device);
    (void)hipFree(b->ptr);
  }
  delete b;
}

template <typename T>
T *unwrap_external(napi_env env, napi_value v) {
  void *p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok) return nullptr;
  return static_cast<T *>(p);
}

// create(device, vocabMax, rowsMax, kMax) -> external
napi_value Create(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return fail(env, "create(device, vocabMax, rowsMax, kMax)");
  int64_t a[4];
  for (int i = 0; i < 4; ++i)
    if (!get_i64(env, argv[i], &a[i]) || !in_i32(a[i], INT32_MIN))
      return fail(env, "create: 32-bit integer arguments expected");
  tabby_sampler *s = nullptr;
  const int rc = tabby_sampler_create((int)a[0], (int32_t)a[1], (int32_t)a[2], (int32_t)a[3], &s);
  if (rc) return fail(env, tabby_last_error());
  Handle *h = new Handle{};
  h->sampler = s;
  h->device = (int)a[0];
  napi_value out;
  CHECK_NAPI(env, napi_create_external(env, h, finalize_handle, nullptr, &out));
  return out;
}

// destroy(handle): frees the scratch now rather than at garbage collection.
napi_value Destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return fail(env, "destroy(handle)");
  Handle *h = unwrap_external<Handle>(env, argv[0]);
  if (!h) return fail(env, "destroy: not a sampler handle");
  release_handle(h);
  return nullptr;
}

// deviceAlloc(device, bytes) -> external
napi_value DeviceAlloc(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return fail(env, "deviceAlloc(device, bytes)");
  int64_t device, bytes;
  if (!get_i64(env, argv[0], &device) || !get_i64(env, argv[1], &bytes) || bytes <= 0)
    return fail(env, "deviceAlloc: device and a positive byte count expected");
  if (hipSetDevice((int)device) != hipSuccess) return fail(env, "deviceAlloc: hipSetDevice failed");
  DeviceBuffer *b = new DeviceBuffer{nullptr, (size_t)bytes, (int)device};
  if (hipMalloc(&b->ptr, b->bytes) != hipSuccess) {
    delete b;
    return fail(env, "deviceAlloc: hipMalloc of " + std::to_string(bytes) + " bytes failed");
  }
  napi_value out;
  CHECK_NAPI(env, napi_create_external(env, b, finalize_buffer, nullptr, &out));
  return out;
}

napi_value DeviceFree(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return fail(env, "deviceFree(buffer)");
  DeviceBuffer *b = unwrap_external<DeviceBuffer>(env, argv[0]);
  if (!b) return fail(env, "deviceFree: not a device buffer");
  if (b->ptr && b->owned) {
    (void)hipSetDevice(b->device);
    (void)hipFree(b->ptr);
  }
  b->ptr = nullptr;
  b->bytes = 0;
  return nullptr;
}

// wrapDevicePointer(device, address: BigInt, bytes) -> external over memory the caller owns
// (e.g. logits a HIP forward pass wrote in this process); the addon never frees it.
napi_value WrapDevicePointer(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return fail(env, "wrapDevicePointer(device, address, bytes)");
  int64_t device, bytes;
  uint64_t address = 0;
  bool lossless = false;
  if (!get_i64(env, argv[0], &device) || !get_i64(env, argv[2], &bytes) || bytes <= 0)
    return fail(env, "wrapDevicePointer: device and a positive byte count expected");
  if (napi_get_value_bigint_uint64(env, argv[1], &address, &lossless) != napi_ok || !lossless ||
      address == 0)
    return fail(env, "wrapDevicePointer: the address must be a nonzero BigInt");
  DeviceBuffer *b = new DeviceBuffer{reinterpret_cast<void *>(address), (size_t)bytes, (int)device, false};
  napi_value out;
  CHECK_NAPI(env, napi_create_external(env, b, finalize_buffer, nullptr, &out));
  return out;
}

// upload(buffer, typedArray): synchronous host -> device copy of the array's bytes.
napi_value Upload(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return fail(env, "upload(buffer, typedArray)");
  DeviceBuffer *b = unwrap_external<DeviceBuffer>(env, argv[0]);
  if (!b || !b->ptr) return fail(env, "upload: not a live device buffer");
  napi_typedarray_type type;
  size_t length;
  void *data;
  napi_value ab;
  size_t offset;
  if (napi_get_typedarray_info(env, argv[1], &type, &length, &data, &ab, &offset) != napi_ok)
    return fail(env, "upload: a typed array is expected");
  size_t elem = 0;
  switch (type) {
    case napi_float32_array: elem = 4; break;
    case napi_uint16_array: elem = 2; break;
    default: return fail(env, "upload: Float32Array (f32) or Uint16Array (f16 bits) expected");
  }
  const size_t bytes = length * elem;
  if (bytes > b->bytes) return fail(env, "upload: the array is larger than the device buffer");
  (void)hipSetDevice(b->device);
  if (hipMemcpy(b->ptr, data, bytes, hipMemcpyHostToDevice) != hipSuccess)
    return fail(env, "upload: hipMemcpy failed");
  return nullptr;
}

napi_value throw_status(napi_env env, int rc) {
  napi_value err, msg, code;
  CHECK_NAPI(env, napi_create_string_utf8(env, tabby_last_error(), NAPI_AUTO_LENGTH, &msg));
  CHECK_NAPI(env, napi_create_error(env, nullptr, msg, &err));
  CHECK_NAPI(env, napi_create_int32(env, rc, &code));
  CHECK_NAPI(env, napi_set_named_property(env, err, "status", code));
  napi_throw(env, err);
  return nullptr;
}

// sample(handle, buffer, dtype, rows, vocab, paramsBytes, topkCap)
//   -> { results: ArrayBuffer(rows*48), topkIds: Int32Array|null, topkLogits: Float32Array|null }
napi_value Sample(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (!get_args(env, info, 7, argv))
    return fail(env, "sample(handle, buffer, dtype, rows, vocab, params, topkCap)");
  Handle *h = unwrap_external<Handle>(env, argv[0]);
  if (!h || !h->sampler) return fail(env, "sample: the sampler was destroyed");
  DeviceBuffer *b = unwrap_external<DeviceBuffer>(env, argv[1]);
  if (!b || !b->ptr) return fail(env, "sample: not a live device buffer");
  int64_t dtype, rows, vocab, cap;
  if (!get_i64(env, argv[2], &dtype) || !get_i64(env, argv[3], &rows) ||
      !get_i64(env, argv[4], &vocab) || !get_i64(env, argv[6], &cap))
    return fail(env, "sample: integer dtype, rows, vocab and topkCap expected");
  if (!in_i32(rows, 1) || !in_i32(vocab, 1) || !in_i32(cap, 0))
    return fail(env, "sample: rows and vocab must be in [1, 2^31 - 1], topkCap in [0, 2^31 - 1]");
  const size_t elem = dtype == TABBY_F16 ? 2 : 4;
  if (!dims_fit(rows, vocab, elem, b->bytes)) return fail(env, "sample: rows x vocab exceeds the device buffer");
  if (cap > 0 && !dims_fit(rows, cap, 4, SIZE_MAX / 2)) return fail(env, "sample: rows x topkCap is too large");
  void *pdata;
  size_t plen;
  if (napi_get_arraybuffer_info(env, argv[5], &pdata, &plen) != napi_ok ||
      plen != (size_t)rows * sizeof(tabby_row_params))
    return fail(env, "sample: params must be an ArrayBuffer of rows x 32 bytes");

  napi_value results_ab, ids_ab = nullptr, logits_ab = nullptr;
  void *res_ptr, *ids_ptr = nullptr, *logits_ptr = nullptr;
  CHECK_NAPI(env, napi_create_arraybuffer(env, (size_t)rows * sizeof(tabby_row_result), &res_ptr, &results_ab));
  if (cap > 0) {
    CHECK_NAPI(env, napi_create_arraybuffer(env, (size_t)rows * cap * 4, &ids_ptr, &ids_ab));
    CHECK_NAPI(env, napi_create_arraybuffer(env, (size_t)rows * cap * 4, &logits_ptr, &logits_ab));
  }
  const int rc = tabby_sampler_sample(h->sampler, b->ptr, (int32_t)dtype, (int32_t)rows,
                                      (int32_t)vocab, static_cast<const tabby_row_params *>(pdata),
                                      static_cast<tabby_row_result *>(res_ptr),
                                      static_cast<int32_t *>(ids_ptr), static_cast<float *>(logits_ptr),
                                      (int32_t)cap, nullptr);
  if (rc) return throw_status(env, rc);
  napi_value out, ids = nullptr, logits = nullptr, null_value;
  CHECK_NAPI(env, napi_create_object(env, &out));
  CHECK_NAPI(env, napi_get_null(env, &null_value));
  CHECK_NAPI(env, napi_set_named_property(env, out, "results", results_ab));
  if (cap > 0) {
    CHECK_NAPI(env, napi_create_typedarray(env, napi_int32_array, (size_t)rows * cap, ids_ab, 0, &ids));
    CHECK_NAPI(env, napi_create_typedarray(env, napi_float32_array, (size_t)rows * cap, logits_ab, 0, &logits));
  }
  CHECK_NAPI(env, napi_set_named_property(env, out, "topkIds", ids ? ids : null_value));
  CHECK_NAPI(env, napi_set_named_property(env, out, "topkLogits", logits ? logits : null_value));
  return out;
}

// argmax(handle, buffer, dtype, rows, vocab) -> Int32Array(rows): one launch, then the ids
// read back (rows x 4 bytes).
napi_value Argmax(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return fail(env, "argmax(handle, buffer, dtype, rows, vocab)");
  Handle *h = unwrap_external<Handle>(env, argv[0]);
  if (!h || !h->sampler) return fail(env, "argmax: the sampler was destroyed");
  DeviceBuffer *b = unwrap_external<DeviceBuffer>(env, argv[1]);
  if (!b || !b->ptr) return fail(env, "argmax: not a live device buffer");
  int64_t dtype, rows, vocab;
  if (!get_i64(env, argv[2], &dtype) || !get_i64(env, argv[3], &rows) || !get_i64(env, argv[4], &vocab))
    return fail(env, "argmax: integer dtype, rows and vocab expected");
  if (!in_i32(rows, 1) || !in_i32(vocab, 1)) return fail(env, "argmax: rows and vocab must be in [1, 2^31 - 1]");
  const size_t elem = dtype == TABBY_F16 ? 2 : 4;
  if (!dims_fit(rows, vocab, elem, b->bytes)) return fail(env, "argmax: rows x vocab exceeds the device buffer");
  if ((size_t)rows > h->ids_cap) {
    (void)hipSetDevice(h->device);
    if (h->ids_dev) (void)hipFree(h->ids_dev);
    h->ids_dev = nullptr;
    h->ids_cap = 0;
    if (hipMalloc((void **)&h->ids_dev, (size_t)rows * sizeof(int32_t)) != hipSuccess)
      return fail(env, "argmax: hipMalloc failed");
    h->ids_cap = (size_t)rows;
  }
  const int rc = tabby_argmax_device(h->sampler, b->ptr, (int32_t)dtype, (int32_t)rows, (int32_t)vocab,
                                     h->ids_dev, nullptr, nullptr);
  if (rc) return throw_status(env, rc);
  napi_value ab, out;
  void *host;
  CHECK_NAPI(env, napi_create_arraybuffer(env, (size_t)rows * 4, &host, &ab));
  if (hipMemcpy(host, h->ids_dev, (size_t)rows * 4, hipMemcpyDeviceToHost) != hipSuccess)
    return fail(env, "argmax: reading the ids back failed");
  CHECK_NAPI(env, napi_create_typedarray(env, napi_int32_array, (size_t)rows, ab, 0, &out));
  return out;
}

// softmaxRows(inBuffer, outBuffer, nRows, rowLen, causalPeriod, causalOffset): on the device,
// in place when both are the same buffer; returns when it is done.
napi_value SoftmaxRows(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  if (!get_args(env, info, 6, argv))
    return fail(env, "softmaxRows(inBuffer, outBuffer, nRows, rowLen, causalPeriod, causalOffset)");
  DeviceBuffer *in = unwrap_external<DeviceBuffer>(env, argv[0]);
  DeviceBuffer *out = unwrap_external<DeviceBuffer>(env, argv[1]);
  if (!in || !in->ptr || !out || !out->ptr) return fail(env, "softmaxRows: not a live device buffer");
  int64_t a[4];
  for (int i = 0; i < 4; ++i)
    if (!get_i64(env, argv[2 + i], &a[i])) return fail(env, "softmaxRows: integer arguments expected");
  if (!in_i32(a[0], 1) || !in_i32(a[1], 1)) return fail(env, "softmaxRows: nRows and rowLen must be in [1, 2^31 - 1]");
  if (!in_i32(a[2], INT32_MIN) || !in_i32(a[3], INT32_MIN))
    return fail(env, "softmaxRows: causalPeriod and causalOffset must be 32-bit integers");
  if (!dims_fit(a[0], a[1], 4, std::min(in->bytes, out->bytes)))
    return fail(env, "softmaxRows: nRows x rowLen exceeds a buffer");
  (void)hipSetDevice(in->device);
  const int rc = tabby_softmax_rows_device(static_cast<const float *>(in->ptr), static_cast<float *>(out->ptr),
                                           (int32_t)a[0], (int32_t)a[1], (int32_t)a[2], (int32_t)a[3], nullptr);
  if (rc) return throw_status(env, rc);
  if (hipStreamSynchronize(nullptr) != hipSuccess) return fail(env, "softmaxRows: the kernel failed");
  return nullptr;
}

// download(buffer, typedArray): synchronous device -> host copy into the array's bytes.
napi_value Download(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return fail(env, "download(buffer, typedArray)");
  DeviceBuffer *b = unwrap_external<DeviceBuffer>(env, argv[0]);
  if (!b || !b->ptr) return fail(env, "download: not a live device buffer");
  napi_typedarray_type type;
  size_t length;
  void *data;
  napi_value ab;
  size_t offset;
  if (napi_get_typedarray_info(env, argv[1], &type, &length, &data, &ab, &offset) != napi_ok)
    return fail(env, "download: a typed array is expected");
  size_t elem = 0;
  switch (type) {
    case napi_float32_array: case napi_int32_array: case napi_uint32_array: elem = 4; break;
    case napi_uint16_array: elem = 2; break;
    default: return fail(env, "download: a 16- or 32-bit typed array is expected");
  }
  const size_t bytes = length * elem;
  if (bytes > b->bytes) return fail(env, "download: the array is larger than the device buffer");
  (void)hipSetDevice(b->device);
  if (hipMemcpy(data, b->ptr, bytes, hipMemcpyDeviceToHost) != hipSuccess)
    return fail(env, "download: hipMemcpy failed");
  return nullptr;
}

napi_value Version(napi_env env, napi_callback_info) {
  napi_value out;
  CHECK_NAPI(env, napi_create_string_utf8(env, tabby_version(), NAPI_AUTO_LENGTH, &out));
  return out;
}

napi_value Init(napi_env env, napi_value exports) {
  const napi_property_descriptor props[] = {
      {"create", nullptr, Create, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"destroy", nullptr, Destroy, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"deviceAlloc", nullptr, DeviceAlloc, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"deviceFree", nullptr, DeviceFree, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"wrapDevicePointer", nullptr, WrapDevicePointer, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"upload", nullptr, Upload, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"sample", nullptr, Sample, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"argmax", nullptr, Argmax, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"softmaxRows", nullptr, SoftmaxRows, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"download", nullptr, Download, nullptr, nullptr, nullptr, napi_default, nullptr},
      {"version", nullptr, Version, nullptr, nullptr, nullptr, napi_default, nullptr},
  };
  if (napi_define_properties(env, exports, sizeof props / sizeof props[0], props) != napi_ok)
    return nullptr;
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
