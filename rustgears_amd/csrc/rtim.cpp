// rtim.cpp — the reference's portable inference-graph file (.rtim):
// magic "RTIM", u32 layer count, then per layer a u32 tag and little-endian
// fields (save_layers / load_inference_layers, src/save.rs:172-279):
//   1 Linear   u32 in, u32 out, f32vec weight, f32vec bias
//   2 Conv2d   u32 in, out, kernel, stride, padding, f32vec weight, bias
//   3 ChannelAffine f32vec scale, f32vec shift
//   4 MaxPool2d u32 kernel, u32 stride      5 Flatten
//   6 Activation u32 code (0..5), f32 param 7 Softmax
// where f32vec is a u32 length followed by that many f32.  Activation code 6
// (SiLU) is this provider's extension; any other unknown code or tag is an
// InvalidData error as in the reference (save.rs:259-267, 272-274).
// Saving writes a temporary file in the target directory and renames it over
// the destination (write_atomic, save.rs:21-32).
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/rgnpu.h"

namespace rgnpu {
extern thread_local std::string g_last_error;
}

struct rgnpu_rtim {
  std::vector<rgnpu_layer> layers;
  std::vector<std::unique_ptr<std::vector<float>>> arrays;
};

namespace {

struct Reader {
  FILE* f;
  bool ok = true;
  uint32_t u32() {
    unsigned char b[4];
    if (ok && fread(b, 1, 4, f) != 4) ok = false;
    return ok ? (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24) : 0;
  }
  float f32() {
    uint32_t u = u32();
    float v;
    std::memcpy(&v, &u, 4);
    return v;
  }
};

struct Writer {
  FILE* f;
  bool ok = true;
  void u32(uint32_t v) {
    unsigned char b[4] = {(unsigned char)v, (unsigned char)(v >> 8), (unsigned char)(v >> 16), (unsigned char)(v >> 24)};
    if (ok && fwrite(b, 1, 4, f) != 4) ok = false;
  }
  void f32(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    u32(u);
  }
  void vec(const float* p, int64_t n) {
    u32((uint32_t)n);
    for (int64_t i = 0; i < n; i++) f32(p[i]);
  }
};

}  // namespace

extern "C" {

int rgnpu_rtim_load(const char* path, rgnpu_rtim** out_handle, const rgnpu_layer** layers, int64_t* n_layers) {
  if (!path || !out_handle || !layers || !n_layers) {
    rgnpu::g_last_error = "NULL argument";
    return RGNPU_ERR_INVALID;
  }
  *out_handle = nullptr;
  FILE* f = fopen(path, "rb");
  if (!f) {
    rgnpu::g_last_error = std::string("cannot open ") + path;
    return RGNPU_ERR_IO;
  }
  auto h = std::make_unique<rgnpu_rtim>();
  Reader r{f};
  int status = RGNPU_OK;
  std::string err;
  auto vec = [&]() -> const float* {
    const uint32_t n = r.u32();
    auto v = std::make_unique<std::vector<float>>();
    for (uint32_t i = 0; i < n && r.ok; i++) v->push_back(r.f32());
    const float* p = v->data();
    h->arrays.push_back(std::move(v));
    return p;
  };
  char magic[4];
  if (fread(magic, 1, 4, f) != 4) {
    status = RGNPU_ERR_IO;
    err = "unexpected end of file";
  } else if (std::memcmp(magic, "RTIM", 4) != 0) {
    status = RGNPU_ERR_FORMAT;
    err = "invalid RTIM model header";
  } else {
    const uint32_t count = r.u32();
    for (uint32_t i = 0; i < count && r.ok && status == RGNPU_OK; i++) {
      rgnpu_layer L{};
      const uint32_t tag = r.u32();
      if (!r.ok) break;
      switch (tag) {
        case 1:  // u32 fields read as the reference's usize: every value fits the int64 fields
          L.kind = RGNPU_LAYER_LINEAR;
          L.in_features = r.u32();
          L.out_features = r.u32();
          L.weight = vec();
          L.weight_len = (int64_t)h->arrays.back()->size();
          L.bias = vec();
          L.bias_len = (int64_t)h->arrays.back()->size();
          break;
        case 2:
          L.kind = RGNPU_LAYER_CONV2D;
          L.in_channels = r.u32();
          L.out_channels = r.u32();
          L.kernel = r.u32();
          L.stride = r.u32();
          L.padding = r.u32();
          L.weight = vec();
          L.weight_len = (int64_t)h->arrays.back()->size();
          L.bias = vec();
          L.bias_len = (int64_t)h->arrays.back()->size();
          break;
        case 3:  // two independent vectors, lengths not compared (save.rs:254)
          L.kind = RGNPU_LAYER_CHANNEL_AFFINE;
          L.scale = vec();
          L.scale_len = (int64_t)h->arrays.back()->size();
          L.shift = vec();
          L.shift_len = (int64_t)h->arrays.back()->size();
          break;
        case 4:
          L.kind = RGNPU_LAYER_MAXPOOL2D;
          L.pool_kernel = r.u32();
          L.pool_stride = r.u32();
          break;
        case 5:
          L.kind = RGNPU_LAYER_FLATTEN;
          break;
        case 6: {
          L.kind = RGNPU_LAYER_ACTIVATION;
          const uint32_t code = r.u32();
          L.act_param = r.f32();
          // Codes 0..5 only, as save.rs:259-267 reads them: SiLU (code 6 in
          // this library's enum) has no RTIM code, so a file carrying it is
          // InvalidData here exactly as it is for the reference.
          if (r.ok && code > 5) {
            status = RGNPU_ERR_FORMAT;
            err = "unknown activation tag " + std::to_string(code);
          }
          L.act = (int32_t)code;
          if (code != 5) L.act_param = 0.0f;
          break;
        }
        case 7:
          L.kind = RGNPU_LAYER_SOFTMAX;
          break;
        default:
          status = RGNPU_ERR_FORMAT;
          err = "unknown layer tag " + std::to_string(tag);
      }
      if (status == RGNPU_OK && r.ok) h->layers.push_back(L);
    }
    if (status == RGNPU_OK && !r.ok) {
      status = RGNPU_ERR_IO;
      err = "unexpected end of file";
    }
  }
  fclose(f);
  if (status != RGNPU_OK) {
    rgnpu::g_last_error = err;
    return status;
  }
  *layers = h->layers.data();
  *n_layers = (int64_t)h->layers.size();
  *out_handle = h.release();
  return RGNPU_OK;
}

void rgnpu_rtim_free(rgnpu_rtim* h) { delete h; }

int rgnpu_rtim_save(const char* path, const rgnpu_layer* layers, int64_t n_layers) {
  if (!path || (n_layers > 0 && !layers) || n_layers < 0) {
    rgnpu::g_last_error = "invalid arguments";
    return RGNPU_ERR_INVALID;
  }
  std::string p(path);
  const size_t slash = p.find_last_of('/');
  const std::string dir = slash == std::string::npos ? "." : (slash == 0 ? "/" : p.substr(0, slash));
  std::string tmpl = dir + "/.rtim-XXXXXX";
  std::vector<char> t(tmpl.begin(), tmpl.end());
  t.push_back('\0');
  const int fd = mkstemp(t.data());
  if (fd < 0) {
    rgnpu::g_last_error = "cannot create temporary file in " + dir;
    return RGNPU_ERR_IO;
  }
  FILE* f = fdopen(fd, "wb");
  if (!f) {
    close(fd);
    unlink(t.data());
    rgnpu::g_last_error = "fdopen failed";
    return RGNPU_ERR_IO;
  }
  Writer w{f};
  if (fwrite("RTIM", 1, 4, f) != 4) w.ok = false;
  w.u32((uint32_t)n_layers);
  int status = RGNPU_OK;
  for (int64_t i = 0; i < n_layers && w.ok; i++) {
    const rgnpu_layer& L = layers[i];
    switch (L.kind) {
      case RGNPU_LAYER_LINEAR:
        w.u32(1); w.u32((uint32_t)L.in_features); w.u32((uint32_t)L.out_features);
        w.vec(L.weight, L.weight_len); w.vec(L.bias, L.bias_len);
        break;
      case RGNPU_LAYER_CONV2D:
        w.u32(2); w.u32((uint32_t)L.in_channels); w.u32((uint32_t)L.out_channels); w.u32((uint32_t)L.kernel);
        w.u32((uint32_t)L.stride); w.u32((uint32_t)L.padding);
        w.vec(L.weight, L.weight_len); w.vec(L.bias, L.bias_len);
        break;
      case RGNPU_LAYER_CHANNEL_AFFINE:
        w.u32(3); w.vec(L.scale, L.scale_len); w.vec(L.shift, L.shift_len);
        break;
      case RGNPU_LAYER_MAXPOOL2D:
        w.u32(4); w.u32((uint32_t)L.pool_kernel); w.u32((uint32_t)L.pool_stride);
        break;
      case RGNPU_LAYER_FLATTEN: w.u32(5); break;
      case RGNPU_LAYER_ACTIVATION:
        // save.rs:209-216 writes codes 0..5; a SiLU layer has none, and a file
        // holding one could not be read by the reference, so it is refused.
        if (L.act < RGNPU_ACT_NONE || L.act > RGNPU_ACT_LEAKY_RELU) {
          status = RGNPU_ERR_INVALID;
          break;
        }
        w.u32(6); w.u32((uint32_t)L.act); w.f32(L.act == RGNPU_ACT_LEAKY_RELU ? L.act_param : 0.0f);
        break;
      case RGNPU_LAYER_SOFTMAX: w.u32(7); break;
      default: status = RGNPU_ERR_INVALID;
    }
  }
  const bool flushed = fflush(f) == 0 && fsync(fileno(f)) == 0;
  fclose(f);
  if (status != RGNPU_OK || !w.ok || !flushed) {
    unlink(t.data());
    rgnpu::g_last_error = status != RGNPU_OK ? "layer has no RTIM encoding (unknown kind, or SiLU, which the "
                                               "reference format cannot hold)"
                                             : "write failed";
    return status != RGNPU_OK ? status : RGNPU_ERR_IO;
  }
  if (rename(t.data(), path) != 0) {
    unlink(t.data());
    rgnpu::g_last_error = std::string("cannot rename onto ") + path;
    return RGNPU_ERR_IO;
  }
  return RGNPU_OK;
}

}  // extern "C"
