// weights.hip -- strict safetensors loads into host or device buffers
// (include/rustral_model.h, rkv_st_*).  The file is memory-mapped
// (safetensors.cpp) and each tensor's bytes go to their destination with one
// copy: memcpy for host buffers, hipMemcpyAsync on the caller's stream for
// device buffers (the call returns after the stream has finished them).
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

#include "../../include/rustral_kv.h"
#include "../../include/rustral_model.h"
#include "safetensors.hpp"

namespace rkv {
void set_error(const std::string& msg);
void clear_error();

int copy_tensors(const st::File& f, const std::vector<const st::Tensor*>& found,
                 const std::vector<void*>& dsts, bool on_device, hipStream_t stream,
                 const char* what) {
  for (size_t i = 0; i < found.size(); ++i) {
    const uint8_t* src = f.data + found[i]->begin;
    const size_t bytes = (size_t)(found[i]->end - found[i]->begin);
    if (bytes == 0) continue;
    if (!on_device) {
      std::memcpy(dsts[i], src, bytes);
    } else if (hipMemcpyAsync(dsts[i], src, bytes, hipMemcpyHostToDevice, stream) != hipSuccess) {
      set_error(std::string(what) + ": upload of '" + found[i]->name + "' failed");
      return RKV_ERR_HIP;
    }
  }
  if (on_device && hipStreamSynchronize(stream) != hipSuccess) {
    set_error(std::string(what) + ": stream synchronisation failed");
    return RKV_ERR_HIP;
  }
  return RKV_OK;
}
}  // namespace rkv

extern "C" int rkv_st_load(const rkv_st_file* f, int n, const char* const* names,
                           const int* ndims, const int64_t* shapes, void* const* dsts,
                           int dst_on_device, void* stream) {
  rkv::clear_error();
  if (!f || n < 0 || (n > 0 && (!names || !ndims || !dsts))) {
    rkv::set_error("rkv_st_load: bad argument");
    return RKV_ERR_INVALID_ARG;
  }
  std::vector<rkv::st::Want> want((size_t)n);
  std::vector<void*> dst((size_t)n);
  size_t o = 0;
  for (int i = 0; i < n; ++i) {
    if (!names[i] || ndims[i] < 0 || ndims[i] > 8 || (ndims[i] > 0 && !shapes) || !dsts[i]) {
      rkv::set_error("rkv_st_load: bad name, shape or destination at index " + std::to_string(i));
      return RKV_ERR_INVALID_ARG;
    }
    want[(size_t)i].name = names[i];
    want[(size_t)i].shape.assign(shapes + o, shapes + o + ndims[i]);
    o += (size_t)ndims[i];
    dst[(size_t)i] = dsts[i];
  }
  std::vector<const rkv::st::Tensor*> found;
  std::string err;
  if (!rkv::st::match(*f->f, want, found, err)) {
    rkv::set_error(err);
    return RKV_ERR_INVALID_ARG;
  }
  return rkv::copy_tensors(*f->f, found, dst, dst_on_device != 0,
                           static_cast<hipStream_t>(stream), "rkv_st_load");
}
