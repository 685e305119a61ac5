// The GGUF reader (fkv_gguf.cpp, host code) under AddressSanitizer and UBSan: random
// truncations, byte flips, 8- and 4-byte field overwrites and insertions of a seed file,
// each opened through fkv_gguf_open and, when accepted, read through every accessor.
// Built and run by tests/test_cpu_gguf_asan.py. The library's error-state helpers are
// given here so the reader links on its own.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <unistd.h>
#include <random>
#include <string>
#include <vector>
#include "ferrum_gguf.h"
#include "fkv_internal.h"
namespace fkv {
static thread_local std::string g_err;
int32_t api_fail(int32_t code, const std::string& msg) { g_err = msg; return code; }
int32_t api_ok() { return 0; }
KeepLastError::KeepLastError() : saved(g_err) {}
KeepLastError::~KeepLastError() { g_err = std::move(saved); }
}  // namespace fkv
int main(int argc, char** argv) {
  FILE* f = fopen(argv[1], "rb");
  std::vector<unsigned char> base(1 << 16);
  base.resize(fread(base.data(), 1, base.size(), f));
  fclose(f);
  const int iters = atoi(argv[2]);
  std::mt19937_64 rng(strtoull(argv[3], nullptr, 10));
  const char* path = argv[4];
  int ok = 0, err = 0;
  for (int it = 0; it < iters; ++it) {
    std::vector<unsigned char> d = base;
    const int kind = it % 5;
    auto r = [&](uint64_t n) { return n ? rng() % n : 0; };
    if (kind == 0) d.resize(r(d.size()));
    else if (kind == 1) { int n = 1 + r(6); while (n--) d[r(d.size())] = (unsigned char)r(256); }
    else if (kind == 2) {
      const uint64_t picks[] = {0, 1, 2, 3, 8, 31, 32, 33, 1ull << 31, 1ull << 32, 1ull << 63,
                                ~0ull, ~0ull - 7, (uint64_t)r(1ull << 32)};
      uint64_t v = picks[r(sizeof(picks) / 8)];
      size_t at = r(d.size() - 8);
      memcpy(&d[at], &v, 8);
    } else if (kind == 3) {
      size_t at = r(d.size());
      std::vector<unsigned char> ins(1 + r(40));
      for (auto& c : ins) c = (unsigned char)r(256);
      d.insert(d.begin() + at, ins.begin(), ins.end());
    } else {  // 4-byte field overwrite
      const uint32_t picks[] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 0x7fffffff, 0xffffffff};
      uint32_t v = picks[r(16)];
      size_t at = r(d.size() - 4);
      memcpy(&d[at], &v, 4);
    }
    FILE* o = fopen(path, "wb");
    fwrite(d.data(), 1, d.size(), o);
    fclose(o);
    fkv_gguf* g = nullptr;
    if (fkv_gguf_open(path, &g) != 0) { ++err; continue; }
    ++ok;
    uint32_t ver; uint64_t al, nm, nt, ds, db;
    fkv_gguf_info(g, &ver, &al, &nm, &nt, &ds, &db);
    for (uint64_t t = 0; t < nt && t < 64; ++t) {
      fkv_gguf_tensor_info ti;
      if (fkv_gguf_tensor(g, t, &ti) == 0) {
        uint64_t idx;
        fkv_gguf_find(g, ti.name, ti.name_len, &idx);
      }
    }
    const char* keys[] = {"general.alignment", "s", "f", "arr", "n", "b", "i", "d", "missing"};
    for (const char* k : keys) {
      fkv_gguf_value v;
      if (fkv_gguf_meta(g, k, strlen(k), &v) == 0 && v.type == 9)
        for (uint64_t e = 0; e < v.count && e < 16; ++e) {
          fkv_gguf_value ev;
          fkv_gguf_meta_array_elem(g, k, strlen(k), e, &ev);
        }
    }
    uint64_t len = 0;
    fkv_gguf_dump(g, nullptr, 0, &len);
    std::vector<char> buf(len + 1);
    fkv_gguf_dump(g, buf.data(), buf.size(), &len);
    fkv_gguf_close(g);
  }
  unlink(path);
  printf("iters %d ok %d err %d\n", iters, ok, err);
  return 0;
}
