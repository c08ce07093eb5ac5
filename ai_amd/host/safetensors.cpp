#include "safetensors.hpp"

#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>

#include "json.hpp"

namespace fiber::safetensors {

struct File::Mapping {
  std::string path;
  void* base = nullptr;
  size_t size = 0;
  const uint8_t* data = nullptr;  // the data section
  size_t data_size = 0;
  ~Mapping() {
    if (base && base != MAP_FAILED) munmap(base, size);
  }
};

int64_t Info::Elements() const {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

int Info::ElementSize() const {
  if (dtype == "F64" || dtype == "I64") return 8;
  if (dtype == "F32" || dtype == "I32") return 4;
  if (dtype == "F16" || dtype == "BF16" || dtype == "I16") return 2;
  if (dtype == "I8" || dtype == "U8" || dtype == "BOOL") return 1;
  return 0;
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
  if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13);  // inf, or NaN with its payload
  } else if (exp == 0) {
    if (man == 0) {
      bits = sign;  // signed zero
    } else {        // subnormal: normalise
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while ((man & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
    }
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

File::File(File&&) noexcept = default;
File& File::operator=(File&&) noexcept = default;
File::~File() = default;

File File::Open(const std::string& path) {
  File f;
  f.add(path);
  return f;
}

File File::OpenDir(const std::string& dir) {
  std::vector<std::string> paths;
  if (DIR* d = opendir(dir.c_str())) {
    while (dirent* e = readdir(d)) {
      const std::string n = e->d_name;
      if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) paths.push_back(dir + "/" + n);
    }
    closedir(d);
  }
  if (paths.empty()) throw Error("safetensors: no *.safetensors in " + dir);
  std::sort(paths.begin(), paths.end());
  File f;
  for (const auto& p : paths) f.add(p);
  const std::string idx = dir + "/model.safetensors.index.json";
  struct stat st;
  if (stat(idx.c_str(), &st) == 0) {
    json::Value v;
    try {
      v = json::parse_file(idx);
    } catch (const json::Error& e) {
      throw Error(std::string("safetensors: index: ") + e.what());
    }
    if (const json::Value* wm = v.find("weight_map")) {
      for (const auto& kv : wm->members()) {
        const std::string& shard = kv.second.as_string();
        auto it = f.entries_.find(kv.first);
        if (it == f.entries_.end())
          throw Error("safetensors: index lists \"" + kv.first + "\" in " + shard + " but no shard holds it");
        const std::string& file = it->second.info.file;
        const std::string base = file.substr(file.find_last_of('/') + 1);
        if (base != shard)
          throw Error("safetensors: index puts \"" + kv.first + "\" in " + shard + ", found in " + base);
      }
    }
  }
  return f;
}

void File::add(const std::string& path) {
  auto m = std::make_unique<Mapping>();
  m->path = path;
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) throw Error("safetensors: cannot open " + path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    throw Error("safetensors: cannot stat " + path);
  }
  m->size = (size_t)st.st_size;
  if (m->size > 0) {
    m->base = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m->base == MAP_FAILED) {
      ::close(fd);
      throw Error("safetensors: cannot map " + path);
    }
  }
  ::close(fd);
  const uint8_t* b = static_cast<const uint8_t*>(m->base);
  if (m->size < 8) throw Error("safetensors: " + path + ": file too short for a header");
  uint64_t n = 0;
  for (int k = 7; k >= 0; k--) n = (n << 8) | b[k];
  if (n > m->size - 8)
    throw Error("safetensors: " + path + ": header length " + std::to_string(n) + " exceeds file size " +
                std::to_string(m->size));
  m->data = b + 8 + n;
  m->data_size = m->size - 8 - n;
  json::Value h;
  try {
    h = json::parse(std::string(reinterpret_cast<const char*>(b + 8), (size_t)n));
  } catch (const json::Error& e) {
    throw Error("safetensors: " + path + ": header: " + e.what());
  }
  if (!h.is_object()) throw Error("safetensors: " + path + ": header is not an object");
  const int src = (int)maps_.size();
  for (const auto& kv : h.members()) {
    const std::string& name = kv.first;
    if (name == "__metadata__") {
      for (const auto& mv : kv.second.members()) meta_[mv.first] = mv.second.as_string();
      continue;
    }
    if (entries_.count(name)) throw Error("safetensors: tensor \"" + name + "\" appears in more than one file");
    Entry e;
    e.src = src;
    e.info.file = path;
    try {
      e.info.dtype = kv.second.at("dtype").as_string();
      for (const auto& d : kv.second.at("shape").items()) e.info.shape.push_back(d.as_int());
      const auto& off = kv.second.at("data_offsets").items();
      if (off.size() != 2) throw json::Error("data_offsets needs two values");
      e.begin = off[0].as_int();
      e.end = off[1].as_int();
    } catch (const json::Error& err) {
      throw Error("safetensors: " + path + ": tensor \"" + name + "\": " + err.what());
    }
    if (e.info.ElementSize() == 0)
      throw Error("safetensors: tensor \"" + name + "\": unknown dtype \"" + e.info.dtype + "\"");
    for (int64_t d : e.info.shape)
      if (d < 0) throw Error("safetensors: tensor \"" + name + "\": negative dimension in its shape");
    if (e.begin < 0 || e.end < e.begin || e.end > (int64_t)m->data_size)
      throw Error("safetensors: tensor \"" + name + "\": data offsets [" + std::to_string(e.begin) + ", " +
                  std::to_string(e.end) + ") outside the data section of " + std::to_string(m->data_size) + " bytes");
    const int64_t want = e.info.Elements() * e.info.ElementSize();
    if (e.end - e.begin != want)
      throw Error("safetensors: tensor \"" + name + "\": " + std::to_string(e.end - e.begin) + " bytes for its shape of " +
                  e.info.dtype + ", want " + std::to_string(want));
    entries_.emplace(name, std::move(e));
  }
  maps_.push_back(std::move(m));
}

std::vector<std::string> File::Names() const {
  std::vector<std::string> n;
  for (const auto& kv : entries_) n.push_back(kv.first);
  return n;
}

const Info* File::Find(const std::string& name) const {
  auto it = entries_.find(name);
  return it == entries_.end() ? nullptr : &it->second.info;
}

const File::Entry& File::entry(const std::string& name) const {
  auto it = entries_.find(name);
  if (it == entries_.end()) throw Error("safetensors: no tensor \"" + name + "\"");
  return it->second;
}

const uint8_t* File::Raw(const std::string& name, size_t* nbytes) const {
  const Entry& e = entry(name);
  *nbytes = (size_t)(e.end - e.begin);
  return maps_[e.src]->data + e.begin;
}

std::vector<float> File::Float32s(const std::string& name) const {
  const Entry& e = entry(name);
  const uint8_t* p = maps_[e.src]->data + e.begin;
  const int64_t n = e.info.Elements();
  std::vector<float> out((size_t)n);
  const std::string& dt = e.info.dtype;
  for (int64_t i = 0; i < n; i++) {
    if (dt == "F32") {
      std::memcpy(&out[i], p + 4 * i, 4);
    } else if (dt == "BF16") {  // exact: bf16 is the top half of an fp32
      const uint32_t bits = (uint32_t)(p[2 * i] | (p[2 * i + 1] << 8)) << 16;
      std::memcpy(&out[i], &bits, 4);
    } else if (dt == "F16") {
      out[i] = f16_to_f32((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
    } else if (dt == "F64") {
      double d;
      std::memcpy(&d, p + 8 * i, 8);
      out[i] = (float)d;
    } else {
      throw Error("safetensors: tensor \"" + name + "\" has dtype " + dt + "; read it with Raw");
    }
  }
  return out;
}

}  // namespace fiber::safetensors
