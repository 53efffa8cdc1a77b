// Packed-weight cache files ("CLFPACK1"): the exact packed codes and scales of
// one weight, keyed by its name, shape, bits, compiler, target and the SHA-256
// of its source bytes and of the packing definition. Same file format and
// checks as src/packed_cache.rs:13-190:
//
//   "CLFPACK1" | u32 LE header length | header JSON | codes | scales
//
// header JSON (compact, field order as written) =
//   {"key":{"name":..,"rows":..,"cols":..,"bits":..,"compiler":..,"target":..,
//           "source_sha256":..,"packing_sha256":..},
//    "codes_sha256":..,"scales_sha256":..}
// file name = hex SHA-256 of the compact key JSON + ".pack". Writes go to a
// temporary file that is renamed into place.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/clef_i4.h"
#include "kernels.hpp"

namespace {

// ---------------------------------------------------------------- SHA-256
// FIPS 180-4, section 6.2.
struct Sha256 {
  uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                   0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
  uint8_t block[64];
  size_t fill = 0;
  uint64_t length = 0;

  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

  void compress(const uint8_t* p) {
    static const uint32_t k[64] = {
        0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
        0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
        0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
        0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
        0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
        0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
        0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
        0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
      w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 | p[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
      const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
      const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
      w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int t = 0; t < 64; ++t) {
      const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[t] + w[t];
      const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
      hh = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    h[0] += a;
    h[1] += b;
    h[2] += c;
    h[3] += d;
    h[4] += e;
    h[5] += f;
    h[6] += g;
    h[7] += hh;
  }

  void update(const void* data, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    length += n;
    if (fill) {
      const size_t take = n < 64 - fill ? n : 64 - fill;
      std::memcpy(block + fill, p, take);
      fill += take;
      p += take;
      n -= take;
      if (fill < 64) return;
      compress(block);
      fill = 0;
    }
    for (; n >= 64; p += 64, n -= 64) compress(p);
    std::memcpy(block, p, n);
    fill = n;
  }

  std::string hex() {
    const uint64_t bits = length * 8;
    const uint8_t one = 0x80, zero = 0;
    update(&one, 1);
    while (fill != 56) update(&zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(len, 8);
    static const char digits[] = "0123456789abcdef";
    std::string out;
    for (uint32_t v : h)
      for (int s = 28; s >= 0; s -= 4) out += digits[(v >> s) & 15];
    return out;
  }
};

std::string sha256_hex(const void* data, size_t n) {
  Sha256 s;
  s.update(data, n);
  return s.hex();
}

// ---------------------------------------------------------------- JSON
// Strings as serde_json writes them: '"' and '\\' escaped, \b \f \n \r \t,
// other control characters as \u00XX, everything else (UTF-8 included) raw.
void put_string(std::string& out, const std::string& s) {
  out += '"';
  for (unsigned char ch : s) {
    switch (ch) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      default:
        if (ch < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof buf, "\\u%04x", ch);
          out += buf;
        } else {
          out += (char)ch;
        }
    }
  }
  out += '"';
}

struct Key {
  std::string name, compiler, target, source_sha256, packing_sha256;
  uint64_t rows = 0, cols = 0, bits = 0;

  std::string json() const {
    std::string o = "{\"name\":";
    put_string(o, name);
    o += ",\"rows\":" + std::to_string(rows) + ",\"cols\":" + std::to_string(cols) +
         ",\"bits\":" + std::to_string(bits) + ",\"compiler\":";
    put_string(o, compiler);
    o += ",\"target\":";
    put_string(o, target);
    o += ",\"source_sha256\":";
    put_string(o, source_sha256);
    o += ",\"packing_sha256\":";
    put_string(o, packing_sha256);
    o += '}';
    return o;
  }
  bool operator==(const Key& k) const {
    return name == k.name && compiler == k.compiler && target == k.target && source_sha256 == k.source_sha256 &&
           packing_sha256 == k.packing_sha256 && rows == k.rows && cols == k.cols && bits == k.bits;
  }
};

// A small reader for the header object: objects, strings, unsigned integers,
// and whitespace between tokens (any valid JSON writer's output for this
// structure). Unknown members are rejected.
struct Parser {
  const char* p;
  const char* end;
  bool ok = true;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool eat(char c) {
    ws();
    if (p < end && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  static int hexval(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }
  std::string str() {
    std::string s;
    if (!eat('"')) {
      ok = false;
      return s;
    }
    while (p < end && *p != '"') {
      if (*p != '\\') {
        s += *p++;
        continue;
      }
      if (++p >= end) break;
      const char e = *p++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp = 0;
          for (int i = 0; i < 4; ++i) {
            const int v = p < end ? hexval(*p++) : -1;
            if (v < 0) {
              ok = false;
              return s;
            }
            cp = cp * 16 + (uint32_t)v;
          }
          if (cp >= 0xD800 && cp < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            uint32_t lo = 0;
            for (int i = 2; i < 6; ++i) {
              const int v = hexval(p[i]);
              if (v < 0) {
                ok = false;
                return s;
              }
              lo = lo * 16 + (uint32_t)v;
            }
            p += 6;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          if (cp < 0x80) {
            s += (char)cp;
          } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 63));
          } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 63));
            s += (char)(0x80 | (cp & 63));
          } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 63));
            s += (char)(0x80 | ((cp >> 6) & 63));
            s += (char)(0x80 | (cp & 63));
          }
          break;
        }
        default: ok = false; return s;
      }
    }
    if (p >= end) ok = false;
    else ++p;
    return s;
  }
  uint64_t num() {
    ws();
    uint64_t v = 0;
    const char* start = p;
    while (p < end && *p >= '0' && *p <= '9') v = v * 10 + (uint64_t)(*p++ - '0');
    if (p == start) ok = false;
    return v;
  }
  Key key() {
    Key k;
    if (!eat('{')) {
      ok = false;
      return k;
    }
    bool first = true;
    while (ok && !eat('}')) {
      if (!first && !eat(',')) {
        ok = false;
        break;
      }
      first = false;
      const std::string f = str();
      if (!eat(':')) {
        ok = false;
        break;
      }
      if (f == "name") k.name = str();
      else if (f == "compiler") k.compiler = str();
      else if (f == "target") k.target = str();
      else if (f == "source_sha256") k.source_sha256 = str();
      else if (f == "packing_sha256") k.packing_sha256 = str();
      else if (f == "rows") k.rows = num();
      else if (f == "cols") k.cols = num();
      else if (f == "bits") k.bits = num();
      else ok = false;
    }
    return k;
  }
};

struct Header {
  Key key;
  std::string codes_sha256, scales_sha256;
};

bool parse_header(const std::string& text, Header& h) {
  Parser ps{text.data(), text.data() + text.size()};
  if (!ps.eat('{')) return false;
  bool first = true;
  while (ps.ok && !ps.eat('}')) {
    if (!first && !ps.eat(',')) return false;
    first = false;
    const std::string f = ps.str();
    if (!ps.eat(':')) return false;
    if (f == "key") h.key = ps.key();
    else if (f == "codes_sha256") h.codes_sha256 = ps.str();
    else if (f == "scales_sha256") h.scales_sha256 = ps.str();
    else return false;
  }
  ps.ws();
  return ps.ok && ps.p == ps.end;
}

// ---------------------------------------------------------------- cache

constexpr char kMagic[8] = {'C', 'L', 'F', 'P', 'A', 'C', 'K', '1'};

int fail(const std::string& msg) { return clef::set_last_error(msg.c_str()); }

// The packing definition the packed bytes depend on: the layout conversion
// (checkpoint 256x64 tiles -> rotated codes in 128x32-word tiles) and the
// quantizer arithmetic of this library (version of csrc/prepare.hip).
const char kPacking[] =
    "tiled256x64-to-rotated-codes128x32-v1\n"
    "clef-hrx_amd gfx950 quantizer: radix-4 strides 1,4,16,64; NaN-as-inf row max; "
    "scale RN(max(RN(m/16),1e-30)/qmax); round-half-even codes; retile 128x32 words\n";

int make_key(const clef_pack_key* in, Key& k) {
  if (!in || !in->name || !in->compiler || !in->target || (!in->source && in->source_bytes))
    return fail("invalid packed-cache key");
  k.name = in->name;
  k.compiler = in->compiler;
  k.target = in->target;
  k.rows = (uint64_t)in->rows;
  k.cols = (uint64_t)in->cols;
  k.bits = (uint64_t)in->bits;
  k.source_sha256 = sha256_hex(in->source, in->source_bytes);
  k.packing_sha256 = sha256_hex(kPacking, sizeof(kPacking) - 1);
  return CLEF_OK;
}

// src/packed_cache.rs:35-55.
int sizes(const Key& k, size_t& codes, size_t& scales) {
  if (!((k.bits == 4 || k.bits == 8) && k.rows > 0 && k.cols > 0 && k.rows % 256 == 0 && k.cols % 256 == 0))
    return fail("invalid packed-cache extent");
  if (k.rows > (uint64_t)1 << 40 || k.cols > (uint64_t)1 << 40 || k.rows * k.cols > ((uint64_t)1 << 60) / k.bits)
    return fail("packed-cache size overflow");
  codes = (size_t)(k.rows * k.cols * k.bits / 8);
  scales = (size_t)(k.rows * 4);
  return CLEF_OK;
}

std::string cache_path(const char* directory, const Key& k) {
  const std::string j = k.json();
  std::string dir = directory;
  if (!dir.empty() && dir.back() != '/') dir += '/';
  return dir + sha256_hex(j.data(), j.size()) + ".pack";
}

bool read_all(int fd, void* dst, size_t n) {
  char* p = static_cast<char*>(dst);
  while (n) {
    const ssize_t r = ::read(fd, p, n);
    if (r <= 0) {
      if (r < 0 && errno == EINTR) continue;
      return false;
    }
    p += r;
    n -= (size_t)r;
  }
  return true;
}

bool write_all(int fd, const void* src, size_t n) {
  const char* p = static_cast<const char*>(src);
  while (n) {
    const ssize_t r = ::write(fd, p, n);
    if (r <= 0) {
      if (r < 0 && errno == EINTR) continue;
      return false;
    }
    p += r;
    n -= (size_t)r;
  }
  return true;
}

int make_dirs(const std::string& dir) {
  std::string acc;
  for (size_t i = 0; i <= dir.size(); ++i) {
    if (i == dir.size() || dir[i] == '/') {
      if (!acc.empty() && ::mkdir(acc.c_str(), 0777) != 0 && errno != EEXIST) return -1;
    }
    if (i < dir.size()) acc += dir[i];
  }
  return 0;
}

struct Fd {
  int fd;
  ~Fd() {
    if (fd >= 0) ::close(fd);
  }
};

}  // namespace

extern "C" {

int clef_pack_cache_path(const char* directory, const clef_pack_key* key, char* path, size_t path_bytes) {
  Key k;
  if (int rc = make_key(key, k)) return rc;
  if (!directory) return fail("invalid packed-cache directory");
  const std::string p = cache_path(directory, k);
  if (!path || path_bytes < p.size() + 1) return fail("packed-cache path buffer too small");
  std::memcpy(path, p.c_str(), p.size() + 1);
  return CLEF_OK;
}

int clef_pack_cache_read(const char* directory, const clef_pack_key* key, void* codes, size_t codes_bytes,
                         void* scales, size_t scales_bytes, int32_t* hit) {
  if (!hit || !directory) return fail("invalid packed-cache arguments");
  *hit = 0;
  Key k;
  if (int rc = make_key(key, k)) return rc;
  const std::string path = cache_path(directory, k);
  Fd f{::open(path.c_str(), O_RDONLY | O_CLOEXEC)};
  if (f.fd < 0) {
    if (errno == ENOENT) return CLEF_OK;  // a miss
    return fail("packed-cache open failed: " + path + ": " + std::strerror(errno));
  }
  size_t code_n, scale_n;
  if (int rc = sizes(k, code_n, scale_n)) return rc;
  char prefix[12];
  if (!read_all(f.fd, prefix, 12)) return fail("truncated packed-cache prefix");
  if (std::memcmp(prefix, kMagic, 8) != 0) return fail("invalid packed-cache magic");
  const uint32_t header_n = (uint32_t)(uint8_t)prefix[8] | (uint32_t)(uint8_t)prefix[9] << 8 |
                            (uint32_t)(uint8_t)prefix[10] << 16 | (uint32_t)(uint8_t)prefix[11] << 24;
  if (header_n > 65536) return fail("oversized packed-cache header");
  struct stat st;
  if (::fstat(f.fd, &st) != 0) return fail("packed-cache stat failed");
  if ((uint64_t)st.st_size != 12u + (uint64_t)header_n + code_n + scale_n) return fail("packed-cache length mismatch");
  std::string text(header_n, '\0');
  if (!read_all(f.fd, &text[0], header_n)) return fail("truncated packed-cache header");
  Header h;
  if (!parse_header(text, h)) return fail("invalid packed-cache header");
  if (!(h.key == k)) return fail("packed-cache key mismatch");
  if (codes_bytes != code_n || scales_bytes != scale_n || !codes || !scales)
    return fail("packed-cache data size mismatch");
  if (!read_all(f.fd, codes, code_n) || !read_all(f.fd, scales, scale_n))
    return fail("truncated packed-cache data");
  if (sha256_hex(codes, code_n) != h.codes_sha256 || sha256_hex(scales, scale_n) != h.scales_sha256)
    return fail("packed-cache checksum mismatch: " + path);
  *hit = 1;
  return CLEF_OK;
}

int clef_pack_cache_write(const char* directory, const clef_pack_key* key, const void* codes, size_t codes_bytes,
                          const void* scales, size_t scales_bytes) {
  if (!directory) return fail("invalid packed-cache arguments");
  Key k;
  if (int rc = make_key(key, k)) return rc;
  size_t code_n, scale_n;
  if (int rc = sizes(k, code_n, scale_n)) return rc;
  if (code_n != codes_bytes || scale_n != scales_bytes || !codes || !scales)
    return fail("packed-cache data size mismatch");
  std::string header = "{\"key\":" + k.json() + ",\"codes_sha256\":";
  put_string(header, sha256_hex(codes, code_n));
  header += ",\"scales_sha256\":";
  put_string(header, sha256_hex(scales, scale_n));
  header += '}';
  if (header.size() > 65536) return fail("oversized packed-cache header");
  if (make_dirs(directory) != 0) return fail(std::string("packed-cache directory: ") + std::strerror(errno));
  const std::string path = cache_path(directory, k);
  static std::atomic<uint64_t> next{0};
  const std::string temporary = path.substr(0, path.size() - 5) + ".tmp." + std::to_string(::getpid()) + "." +
                                std::to_string(next.fetch_add(1));
  Fd f{::open(temporary.c_str(), O_WRONLY | O_CREAT | O_EXCL | O_CLOEXEC, 0644)};
  if (f.fd < 0) return fail("packed-cache create failed: " + temporary + ": " + std::strerror(errno));
  const uint32_t n = (uint32_t)header.size();
  const unsigned char len[4] = {(unsigned char)n, (unsigned char)(n >> 8), (unsigned char)(n >> 16),
                                (unsigned char)(n >> 24)};
  const bool ok = write_all(f.fd, kMagic, 8) && write_all(f.fd, len, 4) && write_all(f.fd, header.data(), n) &&
                  write_all(f.fd, codes, code_n) && write_all(f.fd, scales, scale_n) && ::fsync(f.fd) == 0;
  ::close(f.fd);
  f.fd = -1;
  if (!ok || ::rename(temporary.c_str(), path.c_str()) != 0) {
    const std::string why = std::strerror(errno);
    ::unlink(temporary.c_str());
    return fail("packed-cache write failed: " + path + ": " + why);
  }
  return CLEF_OK;
}

}  // extern "C"
