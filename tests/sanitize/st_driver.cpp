// st_driver.cpp -- host driver for the safetensors reader and writer of
// libq8hip (lama32_mojo_amd/csrc/q8_safetensors.cpp), built with g++ under
// AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_checkpoint_sanitizers.py.  Test infrastructure only.
//
//   st_driver read PATH...          open each file or directory, read every
//                                   tensor and metadata entry; a file that
//                                   fails to open is fine, a crash is not
//   st_driver write PATH            write a small file, read it back, compare
//   st_driver fuzz PATH SEED N      N mutations of the file at PATH (bytes of
//                                   its header flipped, its length prefix
//                                   changed, the file cut short), each opened
//                                   and read like `read`
//
// Exit status 0 when every step ran to its end (opening corrupt files is
// expected to fail with an error code); the sanitizers abort on any
// out-of-bounds access, overflow or undefined behaviour.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/q8hip.h"

namespace {

int read_everything(const char *path) {
  q8_st *st = nullptr;
  if (q8_st_open(path, &st) != Q8_OK) {
    if (std::strlen(q8_st_error()) == 0) {
      std::fprintf(stderr, "%s: failed without a message\n", path);
      return 1;
    }
    return 0;
  }
  const int64_t n = q8_st_count(st);
  std::vector<unsigned char> buf;
  for (int64_t i = 0; i < n; ++i) {
    const char *name = nullptr, *dtype = nullptr, *file = nullptr;
    int ndim = 0;
    const int64_t *shape = nullptr;
    uint64_t begin = 0, nbytes = 0;
    if (q8_st_info(st, i, &name, &dtype, &ndim, &shape, &file, &begin, &nbytes) != Q8_OK) {
      std::fprintf(stderr, "%s: info of tensor %lld failed\n", path, (long long)i);
      q8_st_close(st);
      return 1;
    }
    uint64_t prod = 1;
    for (int d = 0; d < ndim; ++d) prod *= (uint64_t)shape[d];
    (void)prod;
    if (q8_st_find(st, name) < 0) {
      std::fprintf(stderr, "%s: tensor %s not found by name\n", path, name);
      q8_st_close(st);
      return 1;
    }
    if (nbytes > (64u << 20)) continue;
    buf.assign(nbytes + 1, 0);
    (void)q8_st_read(st, i, 0, buf.data(), nbytes);
    (void)q8_st_read(st, i, nbytes, buf.data(), 1);     // past the end: an error
  }
  for (int64_t i = 0; i < q8_st_metadata_count(st); ++i) {
    const char *k = nullptr, *v = nullptr;
    (void)q8_st_metadata(st, i, &k, &v);
  }
  q8_st_close(st);
  return 0;
}

int write_and_read(const char *path) {
  const char *names[3] = {"b.weight", "a\"q\\\xe4\xb8\xad", "empty"};
  const char *dtypes[3] = {"F32", "I8", "F16"};
  const int ndims[3] = {2, 1, 2};
  const int64_t shapes[5] = {3, 4, 5, 0, 7};
  const char *mk[1] = {"format"}, *mv[1] = {"pt"};
  q8_stw *w = nullptr;
  if (q8_stw_open(path, 3, names, dtypes, ndims, shapes, 1, mk, mv, &w) != Q8_OK) return 1;
  float f[12];
  for (int i = 0; i < 12; ++i) f[i] = 0.5f * (float)i;
  const signed char c[5] = {-1, 2, -3, 4, 127};
  if (q8_stw_put(w, 0, f, sizeof f) != Q8_OK || q8_stw_put(w, 1, c, sizeof c) != Q8_OK ||
      q8_stw_put(w, 2, nullptr, 0) != Q8_OK || q8_stw_close(w) != Q8_OK)
    return 1;
  q8_st *st = nullptr;
  if (q8_st_open(path, &st) != Q8_OK) return 1;
  float g[12] = {0};
  const int64_t i = q8_st_find(st, "b.weight");
  const int ok = i >= 0 && q8_st_read(st, i, 0, g, sizeof g) == Q8_OK &&
                 std::memcmp(f, g, sizeof f) == 0;
  q8_st_close(st);
  return ok ? read_everything(path) : 1;
}

int fuzz(const char *path, unsigned seed, int iters) {
  FILE *fp = std::fopen(path, "rb");
  if (!fp) return 1;
  std::vector<unsigned char> src;
  int ch;
  while ((ch = std::fgetc(fp)) != EOF) src.push_back((unsigned char)ch);
  std::fclose(fp);
  if (src.size() < 9) return 1;
  uint64_t hlen = 0;
  std::memcpy(&hlen, src.data(), 8);
  const uint64_t hend = 8 + (hlen < src.size() - 8 ? hlen : src.size() - 8);
  uint64_t x = seed * 2654435761u + 1;
  auto rnd = [&]() {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return x;
  };
  const std::string out = std::string(path) + ".fuzz";
  for (int it = 0; it < iters; ++it) {
    std::vector<unsigned char> b = src;
    switch (rnd() % 4) {
      case 0: {                                   // flip a few header bytes
        const int k = 1 + (int)(rnd() % 4);
        for (int j = 0; j < k; ++j) b[8 + rnd() % (hend - 8)] = (unsigned char)rnd();
        break;
      }
      case 1: {                                   // a structural character in the JSON
        static const char cs[] = "{}[]\",:0-9e.\\ ";
        b[8 + rnd() % (hend - 8)] = (unsigned char)cs[rnd() % (sizeof cs - 1)];
        break;
      }
      case 2: {                                   // another length prefix
        uint64_t v = rnd() % 3 == 0 ? rnd() : hlen + (rnd() % 64) - 32;
        std::memcpy(b.data(), &v, 8);
        break;
      }
      default:                                    // the file cut short
        b.resize(rnd() % b.size());
        break;
    }
    FILE *o = std::fopen(out.c_str(), "wb");
    if (!o) return 1;
    if (!b.empty()) std::fwrite(b.data(), 1, b.size(), o);
    std::fclose(o);
    if (read_everything(out.c_str())) return 1;
  }
  std::remove(out.c_str());
  return 0;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc >= 3 && std::strcmp(argv[1], "read") == 0) {
    for (int i = 2; i < argc; ++i)
      if (read_everything(argv[i])) return 1;
    return 0;
  }
  if (argc == 3 && std::strcmp(argv[1], "write") == 0) return write_and_read(argv[2]);
  if (argc == 5 && std::strcmp(argv[1], "fuzz") == 0)
    return fuzz(argv[2], (unsigned)std::atoi(argv[3]), std::atoi(argv[4]));
  std::fprintf(stderr, "usage: st_driver read PATH... | write PATH | fuzz PATH SEED N\n");
  return 2;
}
