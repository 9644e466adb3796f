// exl3_pack.cpp -- a pack's tensors from its safetensors files, for hosts
// that have no Source of their own (the reference's host, mlx-serve, hands
// the format an MLX Source over the same files:
// turboexl3_ds41/plugin.zig:86-103,127-185; exllamav3 stores a linear as
// <base>.trellis i16 [in/16, out/16, n], <base>.suh f16 [in], <base>.svh f16
// [out]).
//
// safetensors layout: 8 bytes little-endian header length N, N bytes of JSON
// {name: {"dtype", "shape", "data_offsets": [begin, end]}, "__metadata__": ..},
// then the data; offsets count from the end of the header.  Every file is
// mapped read-only and each tensor is handed out as a view into its mapping
// (exl3_host_tensor), valid until the source is closed.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/exl3_mi355x.h"
#include "exl3_json.h"

namespace {

struct Mapping {
  void *base = nullptr;
  size_t bytes = 0;
};

struct Entry {
  const void *data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[EXL3_MAX_DIMS];
};

// exl3_source must stay the first member: the handle is its address.
struct PackSource {
  exl3_source src;
  std::vector<Mapping> maps;
  std::unordered_map<std::string, Entry> tensors;
};

struct PackDir {
  exl3_pack_dir dir;
  std::string root;
};

// safetensors dtype names -> the ABI's dtypes and element sizes; 0 size for
// a name this library has no dtype for.
bool dtype_of(const std::string &s, int32_t *dt, size_t *size) {
  static const struct {
    const char *name;
    int32_t dt;
    size_t size;
  } table[] = {{"BOOL", EXL3_DT_BOOL, 1}, {"U8", EXL3_DT_U8, 1},    {"I8", EXL3_DT_I8, 1},
               {"U16", EXL3_DT_U16, 2},  {"I16", EXL3_DT_I16, 2},  {"F16", EXL3_DT_F16, 2},
               {"BF16", EXL3_DT_BF16, 2}, {"U32", EXL3_DT_U32, 4}, {"I32", EXL3_DT_I32, 4},
               {"F32", EXL3_DT_F32, 4},  {"U64", EXL3_DT_U64, 8},  {"I64", EXL3_DT_I64, 8},
               {"F64", EXL3_DT_F64, 8}};
  for (const auto &e : table)
    if (s == e.name) {
      *dt = e.dt;
      *size = e.size;
      return true;
    }
  return false;
}

int pack_tensor(void *self, exl3_str name, exl3_host_tensor *out) {
  const PackSource *p = static_cast<const PackSource *>(self);
  auto it = p->tensors.find(std::string(name.ptr, name.len));
  if (it == p->tensors.end()) return 0;
  const Entry &e = it->second;
  out->data = e.data;
  out->dtype = e.dtype;
  out->ndim = e.ndim;
  for (int i = 0; i < EXL3_MAX_DIMS; ++i) out->shape[i] = i < e.ndim ? e.shape[i] : 0;
  return 1;
}

uint64_t dir_file_bytes(void *self, exl3_str name) {
  const PackDir *d = static_cast<const PackDir *>(self);
  const std::string rel(name.ptr, name.len);
  if (rel.empty() || rel.find("..") != std::string::npos || rel[0] == '/') return 0;
  struct stat st;
  if (stat((d->root + "/" + rel).c_str(), &st) != 0 || !S_ISREG(st.st_mode)) return 0;
  return (uint64_t)st.st_size;
}

void unmap_all(PackSource *p) {
  for (Mapping &m : p->maps)
    if (m.base) munmap(m.base, m.bytes);
  p->maps.clear();
}

void set_why(exl3_verdict *why, int32_t code, const char *text) {
  if (why) {
    why->code = code;
    why->why = text;
  }
}

// Maps one file and indexes its tensors; a name seen in an earlier file is
// refused (a pack names every tensor once).
bool add_file(PackSource *p, const char *path, exl3_verdict *why) {
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    set_why(why, EXL3_FAILED, "turboexl3_mi355x: a safetensors file cannot be opened");
    return false;
  }
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 8) {
    close(fd);
    set_why(why, EXL3_FAILED, "turboexl3_mi355x: a safetensors file is shorter than its header");
    return false;
  }
  const size_t bytes = (size_t)st.st_size;
  void *base = mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (base == MAP_FAILED) {
    set_why(why, EXL3_FAILED, "turboexl3_mi355x: a safetensors file cannot be mapped");
    return false;
  }
  p->maps.push_back(Mapping{base, bytes});
  const uint8_t *b = static_cast<const uint8_t *>(base);
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | b[i];
  if (n > bytes - 8) {
    set_why(why, EXL3_FAILED, "turboexl3_mi355x: a safetensors header runs past its file");
    return false;
  }
  const exl3::Json h = exl3::Json::parse(reinterpret_cast<const char *>(b + 8), (size_t)n);
  if (!h.is_object()) {
    set_why(why, EXL3_FAILED, "turboexl3_mi355x: a safetensors header is not a JSON object");
    return false;
  }
  const uint8_t *data = b + 8 + n;
  const uint64_t data_bytes = bytes - 8 - n;
  for (const auto &kv : h.obj) {
    if (kv.first == "__metadata__") continue;
    const exl3::Json &t = kv.second;
    const exl3::Json *dt = t.get("dtype"), *shape = t.get("shape"), *off = t.get("data_offsets");
    int32_t code;
    size_t esize;
    if (!dt || dt->kind != exl3::Json::STRING || !dtype_of(dt->str, &code, &esize)) {
      set_why(why, EXL3_UNSUPPORTED, "turboexl3_mi355x: a safetensors tensor of an unknown dtype");
      return false;
    }
    if (!shape || shape->kind != exl3::Json::ARRAY || shape->arr.size() > EXL3_MAX_DIMS || !off ||
        off->kind != exl3::Json::ARRAY || off->arr.size() != 2) {
      set_why(why, EXL3_FAILED, "turboexl3_mi355x: a safetensors tensor entry is malformed");
      return false;
    }
    Entry e{};
    e.dtype = code;
    e.ndim = (int32_t)shape->arr.size();
    uint64_t count = 1;
    for (int i = 0; i < e.ndim; ++i) {
      const exl3::Json &d = shape->arr[i];
      if (d.kind != exl3::Json::NUMBER || !d.integral || d.num < 0 || d.num > 9.0e15) {
        set_why(why, EXL3_FAILED, "turboexl3_mi355x: a safetensors shape is not a list of sizes");
        return false;
      }
      e.shape[i] = (int64_t)d.num;
      count *= (uint64_t)e.shape[i];
    }
    const exl3::Json &o0 = off->arr[0], &o1 = off->arr[1];
    if (o0.kind != exl3::Json::NUMBER || o1.kind != exl3::Json::NUMBER || !o0.integral ||
        !o1.integral || o0.num < 0 || o1.num < o0.num || o1.num > (double)data_bytes ||
        (uint64_t)(o1.num - o0.num) != count * esize) {
      set_why(why, EXL3_FAILED, "turboexl3_mi355x: safetensors data offsets disagree with the file");
      return false;
    }
    e.data = data + (uint64_t)o0.num;
    if (!p->tensors.emplace(kv.first, e).second) {
      set_why(why, EXL3_FAILED, "turboexl3_mi355x: a tensor name appears in two safetensors files");
      return false;
    }
  }
  return true;
}

}  // namespace

extern "C" {

exl3_source *exl3_safetensors_open(const char *const *paths, uint32_t count, exl3_verdict *why) {
  set_why(why, EXL3_OK, "");
  if (paths == nullptr || count == 0) {
    set_why(why, EXL3_FAILED, "turboexl3_mi355x: no safetensors file named");
    return nullptr;
  }
  PackSource *p = new PackSource;
  p->src.self = p;
  p->src.tensor = &pack_tensor;
  for (uint32_t i = 0; i < count; ++i) {
    if (paths[i] == nullptr || !add_file(p, paths[i], why)) {
      if (paths[i] == nullptr) set_why(why, EXL3_FAILED, "turboexl3_mi355x: no safetensors file named");
      unmap_all(p);
      delete p;
      return nullptr;
    }
  }
  return &p->src;
}

void exl3_safetensors_close(exl3_source *src) {
  if (src == nullptr) return;
  PackSource *p = reinterpret_cast<PackSource *>(src);
  unmap_all(p);
  delete p;
}

exl3_pack_dir *exl3_pack_dir_open(const char *root) {
  if (root == nullptr) return nullptr;
  struct stat st;
  if (stat(root, &st) != 0 || !S_ISDIR(st.st_mode)) return nullptr;
  PackDir *d = new PackDir;
  d->dir.self = d;
  d->dir.file_bytes = &dir_file_bytes;
  d->root = root;
  return &d->dir;
}

void exl3_pack_dir_close(exl3_pack_dir *dir) {
  if (dir != nullptr) delete reinterpret_cast<PackDir *>(dir);
}

}  // extern "C"
