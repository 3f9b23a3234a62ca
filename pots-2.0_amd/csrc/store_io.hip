// Stored steps from disk to device memory: the leaf files of the on-disk transcript store,
// which the reference writes with torch.save (verification/transcript/store.py:285-380) and
// reads back one torch.load at a time (store.py:347-357).
//
// A torch.save file is a ZIP archive of stored records (PKWARE APPNOTE.TXT): `<p>/data.pkl`,
// the pickle of the saved object; `<p>/data/<key>`, the bytes of each storage the pickle
// names; and small records such as `<p>/byteorder`. pots_store_scan reads the central
// directory and walks the pickle's opcodes on a small stack, executing nothing. It accepts
// only the program torch.save writes for one plain tensor and reports anything else as
// POTS_STORE_OTHER, which the caller reads with torch.load(weights_only=True) instead.
// pots_store_load then reads the storages' bytes with pread on several host threads into
// pinned staging and sends each filled slot to the device with one hipMemcpyAsync.
//
// Host code only.

#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <string>
#include <thread>
#include <vector>

#include "common.h"

namespace pots {
namespace {

constexpr uint32_t kDefaultThreads = 8;
constexpr uint32_t kMaxThreads = 64;
constexpr uint64_t kMaxPickle = 1u << 16;     // one tensor's pickle is a few hundred bytes
constexpr uint64_t kMaxDirectory = 1u << 24;  // central directory bytes
constexpr uint64_t kMinSlot = 64u << 10;

struct Fd {
  int fd;
  explicit Fd(const char* path) : fd(::open(path, O_RDONLY | O_CLOEXEC)) {}
  ~Fd() {
    if (fd >= 0) ::close(fd);
  }
  Fd(const Fd&) = delete;
  Fd& operator=(const Fd&) = delete;
};

// Exactly n bytes at `off`; false on an error or the end of the file.
bool read_at(int fd, void* dst, uint64_t n, uint64_t off) {
  char* p = static_cast<char*>(dst);
  while (n > 0) {
    const size_t want = (size_t)std::min<uint64_t>(n, 1u << 30);
    const ssize_t r = ::pread(fd, p, want, (off_t)off);
    if (r < 0) {
      if (errno == EINTR) continue;
      return false;
    }
    if (r == 0) return false;
    p += r;
    n -= (uint64_t)r;
    off += (uint64_t)r;
  }
  return true;
}

inline uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | p[1] << 8); }
inline uint32_t le32(const uint8_t* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
inline uint64_t le64(const uint8_t* p) { return le32(p) | (uint64_t)le32(p + 4) << 32; }

// A file being scanned. Its first and last few KiB are read once and reads inside them are
// served from memory: a torch.save archive keeps its small records, their local headers and
// the central directory there, so a scan costs two reads.
struct ScanFile {
  static constexpr uint64_t kWindow = 4096;
  int fd = -1;
  uint64_t size = 0;
  std::vector<uint8_t> head, tail;
  uint64_t tail_off = 0;

  bool open_windows() {
    head.resize(std::min(size, kWindow));
    tail_off = size - std::min(size, kWindow);
    tail.resize(size - tail_off);
    return read_at(fd, head.data(), head.size(), 0) &&
           read_at(fd, tail.data(), tail.size(), tail_off);
  }
  bool read(void* dst, uint64_t n, uint64_t off) const {
    if (n <= head.size() && off <= head.size() - n) {
      memcpy(dst, head.data() + off, n);
      return true;
    }
    if (off >= tail_off && n <= tail.size() && off - tail_off <= tail.size() - n) {
      memcpy(dst, tail.data() + (off - tail_off), n);
      return true;
    }
    return read_at(fd, dst, n, off);
  }
};

// ---- the ZIP directory ---------------------------------------------------------------------

struct Entry {
  std::string name;
  uint32_t method = 0, flags = 0;
  uint64_t csize = 0, usize = 0, local = 0;
  bool dir = false;  // a directory entry (MS-DOS attribute or a trailing '/'): it has no data
};

// The central directory's entries (APPNOTE 4.3.12 and 4.3.16, with the ZIP64 end records of
// 4.3.14-4.3.15 and the ZIP64 extended information extra field of 4.5.3).
bool directory(const ScanFile& f, std::vector<Entry>* out) {
  if (f.size < 22) return false;
  // The end record sits in the last 22 bytes unless a comment (up to 64 KiB) follows it.
  std::vector<uint8_t> big;
  const std::vector<uint8_t>* tailp = &f.tail;
  int64_t e = -1;
  for (int pass = 0; pass < 2 && e < 0; ++pass) {
    if (pass == 1) {
      const uint64_t n = std::min<uint64_t>(f.size, 65535 + 22);
      if (n <= f.tail.size()) break;
      big.resize(n);
      if (!read_at(f.fd, big.data(), n, f.size - n)) return false;
      tailp = &big;
    }
    for (int64_t i = (int64_t)tailp->size() - 22; i >= 0; --i) {
      if (le32(&(*tailp)[i]) == 0x06054b50u) {
        e = i;
        break;
      }
    }
  }
  if (e < 0) return false;
  const std::vector<uint8_t>& tail = *tailp;
  const uint8_t* eo = &tail[e];
  uint64_t n_entries = le16(eo + 10), on_disk = le16(eo + 8), cd_size = le32(eo + 12),
           cd_off = le32(eo + 16), disk = le16(eo + 4), cd_disk = le16(eo + 6);
  // A ZIP64 locator before the end record makes the ZIP64 end record's values the ones that
  // count, whatever the 32-bit record says (torch writes both); one that cannot be followed
  // rejects the file.
  if (e >= 20 && le32(eo - 20) == 0x07064b50u) {
    const uint8_t* loc = eo - 20;
    const uint64_t z_off = le64(loc + 8);
    uint8_t z[56];
    if (f.size < 56 || z_off > f.size - 56 || !f.read(z, 56, z_off) ||
        le32(z) != 0x06064b50u || le64(z + 4) < 44 || le32(loc + 16) != 1)
      return false;
    disk = le32(z + 16);
    cd_disk = le32(z + 20);
    on_disk = le64(z + 24);
    n_entries = le64(z + 32);
    cd_size = le64(z + 40);
    cd_off = le64(z + 48);
  } else if (n_entries == 0xFFFF || cd_size == 0xFFFFFFFFu || cd_off == 0xFFFFFFFFu) {
    return false;
  }
  // One disk only, as torch's ZIP reader requires.
  if (disk != 0 || cd_disk != 0 || on_disk != n_entries || n_entries > 0xFFFFFFFFu) return false;
  if (cd_size > kMaxDirectory || cd_off > f.size || cd_size > f.size - cd_off ||
      cd_size < n_entries * 46)
    return false;
  std::vector<uint8_t> cd(cd_size);
  if (cd_size && !f.read(cd.data(), cd_size, cd_off)) return false;
  out->clear();
  uint64_t p = 0;
  for (uint64_t k = 0; k < n_entries; ++k) {
    if (p + 46 > cd_size || le32(&cd[p]) != 0x02014b50u) return false;
    const uint8_t* h = &cd[p];
    Entry en;
    en.flags = le16(h + 8);
    en.method = le16(h + 10);
    en.csize = le32(h + 20);
    en.usize = le32(h + 24);
    const uint32_t nl = le16(h + 28), xl = le16(h + 30), cl = le16(h + 32);
    en.local = le32(h + 42);
    if (p + 46 + (uint64_t)nl + xl + cl > cd_size) return false;
    en.name.assign(reinterpret_cast<const char*>(h + 46), nl);
    en.dir = (le32(h + 38) & 0x10) || (nl > 0 && en.name.back() == '/');
    // ZIP64 extra field: the 64-bit values of the fields set to all ones, in this order.
    const uint8_t* x = h + 46 + nl;
    for (uint32_t q = 0; q + 4 <= xl;) {
      const uint32_t id = le16(x + q), len = le16(x + q + 2);
      if (q + 4 + len > xl) return false;
      if (id == 0x0001) {
        const uint8_t* v = x + q + 4;
        uint32_t used = 0;
        auto take = [&](uint64_t* f) {
          if (used + 8 > len) return false;
          *f = le64(v + used);
          used += 8;
          return true;
        };
        if (en.usize == 0xFFFFFFFFu && !take(&en.usize)) return false;
        if (en.csize == 0xFFFFFFFFu && !take(&en.csize)) return false;
        if (en.local == 0xFFFFFFFFu && !take(&en.local)) return false;
      }
      q += 4 + len;
    }
    // The entry checks of torch's ZIP reader: no encryption or patch data (flag bits 0, 5, 6
    // and 13), sizes that agree for a stored
    // record, no data without compressed bytes, the first disk, a local header inside the file.
    if ((en.flags & 0x2061) || (en.method == 0 && en.usize != en.csize) ||
        (en.usize && !en.csize) || le16(h + 34) != 0 || en.local > f.size ||
        en.csize > f.size - en.local || f.size - en.local - en.csize < 30)
      return false;
    out->push_back(std::move(en));
    p += 46 + (uint64_t)nl + xl + cl;
  }
  return true;
}

// Where a stored (uncompressed, unencrypted) record's bytes start; false if it is not one.
bool record_data(const ScanFile& f, const Entry& en, uint64_t* data) {
  if (en.dir || en.method != 0 || (en.flags & 1) || en.csize != en.usize) return false;
  uint8_t h[30];
  if (en.local > f.size || f.size - en.local < 30 || !f.read(h, 30, en.local)) return false;
  if (le32(h) != 0x04034b50u) return false;
  const uint64_t start = en.local + 30 + le16(h + 26) + le16(h + 28);
  if (start > f.size || en.usize > f.size - start) return false;
  *data = start;
  return true;
}

// Whether s is well-formed UTF-8 (RFC 3629): torch.load decodes every record name.
bool utf8(const std::string& s) {
  const auto* p = reinterpret_cast<const uint8_t*>(s.data());
  const size_t n = s.size();
  for (size_t i = 0; i < n;) {
    const uint8_t c = p[i];
    size_t len;
    uint32_t cp;
    if (c < 0x80) {
      ++i;
      continue;
    } else if ((c & 0xE0) == 0xC0) {
      len = 2, cp = c & 0x1F;
    } else if ((c & 0xF0) == 0xE0) {
      len = 3, cp = c & 0x0F;
    } else if ((c & 0xF8) == 0xF0) {
      len = 4, cp = c & 0x07;
    } else {
      return false;
    }
    if (i + len > n) return false;
    for (size_t k = 1; k < len; ++k) {
      if ((p[i + k] & 0xC0) != 0x80) return false;
      cp = cp << 6 | (p[i + k] & 0x3F);
    }
    static const uint32_t kMin[5] = {0, 0, 0x80, 0x800, 0x10000};
    if (cp < kMin[len] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
    i += len;
  }
  return true;
}

// ---- the pickle ----------------------------------------------------------------------------

struct Val {
  enum Kind { INT, STR, GLOBAL, TUPLE, MARK, BOOL, ODICT, STORAGE, TENSOR } kind;
  int64_t i = 0;  // INT value, BOOL value, STORAGE numel
  std::string a;  // STR text, GLOBAL module, STORAGE key
  std::string b;  // GLOBAL name
  uint32_t dtype = 0;
  std::vector<Val> items;  // TUPLE items; TENSOR: size tuple, stride tuple
  Val() : kind(INT) {}
  explicit Val(Kind k) : kind(k) {}
};

struct StorageType {
  const char* name;
  uint32_t dtype, esz;
};
constexpr StorageType kStorages[] = {
    {"FloatStorage", POTS_STORE_F32, 4},  {"DoubleStorage", POTS_STORE_F64, 8},
    {"HalfStorage", POTS_STORE_F16, 2},   {"BFloat16Storage", POTS_STORE_BF16, 2},
    {"LongStorage", POTS_STORE_I64, 8},   {"IntStorage", POTS_STORE_I32, 4},
    {"ShortStorage", POTS_STORE_I16, 2},  {"CharStorage", POTS_STORE_I8, 1},
    {"ByteStorage", POTS_STORE_U8, 1},    {"BoolStorage", POTS_STORE_BOOL, 1},
};

uint32_t elem_size(uint32_t dtype) {
  for (const auto& s : kStorages)
    if (s.dtype == dtype) return s.esz;
  return 0;
}

bool all_ints(const Val& t) {
  if (t.kind != Val::TUPLE) return false;
  for (const auto& v : t.items)
    if (v.kind != Val::INT) return false;
  return true;
}

// The tensor torch.save pickled, or false for any other program. Opcodes are those of pickle
// protocols 2-4 (Lib/pickletools.py documents each); memo puts are skipped, and any opcode
// outside this set (memo gets included) rejects the file.
bool parse_pickle(const uint8_t* p, uint64_t n, Val* result) {
  std::vector<Val> st;
  uint64_t i = 0;
  auto need = [&](uint64_t k) { return i + k <= n; };
  auto line = [&](std::string* s) {
    const uint64_t j0 = i;
    while (i < n && p[i] != '\n') ++i;
    if (i >= n) return false;
    s->assign(reinterpret_cast<const char*>(p + j0), i - j0);
    ++i;
    return true;
  };
  auto pop_mark = [&](std::vector<Val>* items) {
    size_t m = st.size();
    while (m > 0 && st[m - 1].kind != Val::MARK) --m;
    if (m == 0) return false;
    items->assign(std::make_move_iterator(st.begin() + m), std::make_move_iterator(st.end()));
    st.resize(m - 1);
    return true;
  };
  auto tuple_of = [&](size_t k) {
    if (st.size() < k) return false;
    Val t(Val::TUPLE);
    t.items.assign(std::make_move_iterator(st.end() - k), std::make_move_iterator(st.end()));
    st.resize(st.size() - k);
    for (const auto& v : t.items)
      if (v.kind == Val::MARK) return false;
    st.push_back(std::move(t));
    return true;
  };
  while (i < n) {
    const uint8_t op = p[i++];
    switch (op) {
      case 0x80:  // PROTO
        if (!need(1) || p[i] < 2 || p[i] > 5) return false;
        ++i;
        break;
      case 'c': {  // GLOBAL
        Val g(Val::GLOBAL);
        if (!line(&g.a) || !line(&g.b)) return false;
        st.push_back(std::move(g));
        break;
      }
      case 'q': case 'r':  // BINPUT, LONG_BINPUT: memoize the top (not through a MARK)
        if (!need(op == 'q' ? 1 : 4) || st.empty() || st.back().kind == Val::MARK) return false;
        i += op == 'q' ? 1 : 4;
        break;
      case '(':  // MARK
        st.emplace_back(Val::MARK);
        break;
      case 'X': case 0x8c: {  // BINUNICODE, SHORT_BINUNICODE
        const uint32_t w = op == 'X' ? 4 : 1;
        if (!need(w)) return false;
        const uint64_t len = w == 4 ? le32(p + i) : p[i];
        i += w;
        if (!need(len)) return false;
        Val s(Val::STR);
        s.a.assign(reinterpret_cast<const char*>(p + i), len);
        i += len;
        if (!utf8(s.a)) return false;
        st.push_back(std::move(s));
        break;
      }
      case 'J': case 'K': case 'M': {  // BININT, BININT1, BININT2
        const uint32_t w = op == 'J' ? 4 : op == 'K' ? 1 : 2;
        if (!need(w)) return false;
        Val v(Val::INT);
        v.i = op == 'J' ? (int64_t)(int32_t)le32(p + i) : op == 'K' ? p[i] : le16(p + i);
        i += w;
        st.push_back(std::move(v));
        break;
      }
      case 0x8a: {  // LONG1: little-endian two's complement of up to 8 bytes here
        if (!need(1)) return false;
        const uint32_t len = p[i++];
        if (len > 8 || !need(len)) return false;
        uint64_t u = 0;
        for (uint32_t k = 0; k < len; ++k) u |= (uint64_t)p[i + k] << (8 * k);
        if (len > 0 && len < 8 && (p[i + len - 1] & 0x80)) u |= ~0ull << (8 * len);
        i += len;
        Val v(Val::INT);
        v.i = (int64_t)u;
        st.push_back(std::move(v));
        break;
      }
      case ')':  // EMPTY_TUPLE
        st.emplace_back(Val::TUPLE);
        break;
      case 0x85: case 0x86: case 0x87:  // TUPLE1, TUPLE2, TUPLE3
        if (!tuple_of(op - 0x84)) return false;
        break;
      case 't': {  // TUPLE
        Val t(Val::TUPLE);
        if (!pop_mark(&t.items)) return false;
        st.push_back(std::move(t));
        break;
      }
      case 0x88: case 0x89: {  // NEWTRUE, NEWFALSE
        Val v(Val::BOOL);
        v.i = op == 0x88;
        st.push_back(std::move(v));
        break;
      }
      case 'Q': {  // BINPERSID: ('storage', torch.<T>Storage, key, location, numel)
        if (st.empty()) return false;
        Val pid = std::move(st.back());
        st.pop_back();
        if (pid.kind != Val::TUPLE || pid.items.size() != 5) return false;
        const auto& it = pid.items;
        if (it[0].kind != Val::STR || it[0].a != "storage" || it[1].kind != Val::GLOBAL ||
            it[1].a != "torch" || it[2].kind != Val::STR || it[3].kind != Val::STR ||
            it[4].kind != Val::INT || it[4].i < 0)
          return false;
        // The device the tensor was saved from; torch.load maps it to the host.
        const std::string& where = it[3].a;
        if (where != "cpu" && where.compare(0, 4, "cuda") != 0) return false;
        if (where.size() > 4 && (where[4] != ':' || where.size() == 5 ||
                                 where.find_first_not_of("0123456789", 5) != std::string::npos))
          return false;
        Val s(Val::STORAGE);
        for (const auto& t : kStorages)
          if (it[1].b == t.name) s.dtype = t.dtype;
        if (s.dtype == 0) return false;
        s.a = it[2].a;
        s.i = it[4].i;
        st.push_back(std::move(s));
        break;
      }
      case 'R': {  // REDUCE
        if (st.size() < 2) return false;
        Val args = std::move(st.back());
        st.pop_back();
        Val fn = std::move(st.back());
        st.pop_back();
        if (fn.kind != Val::GLOBAL || args.kind != Val::TUPLE) return false;
        if (fn.a == "collections" && fn.b == "OrderedDict" && args.items.empty()) {
          st.emplace_back(Val::ODICT);
        } else if (fn.a == "torch._utils" && fn.b == "_rebuild_tensor_v2" &&
                   args.items.size() == 6) {
          auto& a = args.items;
          if (a[0].kind != Val::STORAGE || a[1].kind != Val::INT || !all_ints(a[2]) ||
              !all_ints(a[3]) || a[2].items.size() != a[3].items.size() ||
              a[4].kind != Val::BOOL || a[5].kind != Val::ODICT)
            return false;
          if (a[4].i != 0) return false;  // requires_grad: torch.load would set it
          Val t(Val::TENSOR);
          t.a = a[0].a;
          t.dtype = a[0].dtype;
          t.i = a[0].i;  // storage numel
          t.items.push_back(std::move(a[2]));
          t.items.push_back(std::move(a[3]));
          t.items.push_back(std::move(a[1]));  // storage offset
          st.push_back(std::move(t));
        } else {
          return false;
        }
        break;
      }
      case '.':  // STOP
        if (st.size() != 1 || st[0].kind != Val::TENSOR || i != n) return false;
        *result = std::move(st[0]);
        return true;
      default:
        return false;
    }
  }
  return false;
}

// ---- one file -------------------------------------------------------------------------------

// The whole of a small stored record equals `want`; false if absent, different or unreadable.
bool record_is(const ScanFile& f, const Entry* e, const char* want) {
  const size_t n = strlen(want);
  uint64_t at = 0;
  if (!e || e->usize != n || !record_data(f, *e, &at)) return false;
  char buf[16];
  return n <= sizeof buf && f.read(buf, n, at) && memcmp(buf, want, n) == 0;
}

int32_t scan_one(const char* path, pots_stored_tensor* out) {
  Fd fd(path);
  if (fd.fd < 0) return POTS_STORE_UNREADABLE;
  struct stat sb;
  if (fstat(fd.fd, &sb) != 0 || !S_ISREG(sb.st_mode)) return POTS_STORE_UNREADABLE;
  ScanFile f;
  f.fd = fd.fd;
  f.size = (uint64_t)sb.st_size;
  std::vector<Entry> entries;
  if (!f.open_windows() || !directory(f, &entries) || entries.empty())
    return POTS_STORE_UNREADABLE;
  // torch's reader takes the archive's folder from its first entry, and every record name
  // must lie in that folder and decode as UTF-8.
  const size_t slash = entries[0].name.find('/');
  if (slash == std::string::npos) return POTS_STORE_OTHER;
  const std::string prefix = entries[0].name.substr(0, slash + 1);  // "<p>/"
  for (const auto& e : entries)
    if (!utf8(e.name) || e.name.size() >= 511 || e.name.compare(0, prefix.size(), prefix) != 0)
      return POTS_STORE_OTHER;
  auto find = [&](const std::string& name) -> const Entry* {
    const Entry* hit = nullptr;
    for (const auto& e : entries)
      if (e.name == name) {
        if (hit) return nullptr;
        hit = &e;
      }
    return hit;
  };
  auto has = [&](const std::string& name) {
    for (const auto& e : entries)
      if (e.name == name) return true;
    return false;
  };
  // The small records, exactly as torch.save writes them; any other content goes to
  // torch.load, which decides.
  uint64_t at = 0;
  const std::string ver = has(prefix + ".data/version") ? ".data/version" : "version";
  if (!record_is(f, find(prefix + ver), "3\n")) return POTS_STORE_OTHER;
  if (!record_is(f, find(prefix + "byteorder"), "little")) return POTS_STORE_OTHER;
  if (has(prefix + ".format_version") &&
      !record_is(f, find(prefix + ".format_version"), "1"))
    return POTS_STORE_OTHER;
  if (has(prefix + ".storage_alignment") &&
      !record_is(f, find(prefix + ".storage_alignment"), "64"))
    return POTS_STORE_OTHER;
  if (has(prefix + ".data/serialization_id")) {  // torch reads it as text
    const Entry* id = find(prefix + ".data/serialization_id");
    char buf[256];
    if (!id || id->usize > sizeof buf || !record_data(f, *id, &at) ||
        !f.read(buf, id->usize, at) || !utf8(std::string(buf, id->usize)))
      return POTS_STORE_OTHER;
  }
  const Entry* pkl = find(prefix + "data.pkl");
  if (!pkl) return POTS_STORE_OTHER;
  if (pkl->usize > kMaxPickle || !record_data(f, *pkl, &at)) return POTS_STORE_OTHER;
  std::vector<uint8_t> pk(pkl->usize);
  if (!pk.empty() && !f.read(pk.data(), pk.size(), at)) return POTS_STORE_UNREADABLE;
  Val t(Val::INT);
  if (!parse_pickle(pk.data(), pk.size(), &t)) return POTS_STORE_OTHER;
  const Entry* data = find(prefix + "data/" + t.a);
  if (!data || !record_data(f, *data, &at)) return POTS_STORE_OTHER;

  const uint32_t esz = elem_size(t.dtype);
  const auto& size = t.items[0].items;
  const auto& stride = t.items[1].items;
  const int64_t off = t.items[2].i;
  const uint64_t numel = (uint64_t)t.i;
  if (size.size() > POTS_STORE_MAX_DIM || off < 0) return POTS_STORE_OTHER;
  if (numel > data->usize / esz || numel * esz != data->usize) return POTS_STORE_OTHER;
  // Every element inside the storage; an empty tensor or a negative stride goes to torch.load.
  uint64_t last = (uint64_t)off;
  for (size_t d = 0; d < size.size(); ++d) {
    if (size[d].i <= 0 || stride[d].i < 0) return POTS_STORE_OTHER;
    const unsigned __int128 reach = (unsigned __int128)(uint64_t)(size[d].i - 1) *
                                    (uint64_t)stride[d].i;
    if (reach >= numel) return POTS_STORE_OTHER;
    last += (uint64_t)reach;
    if (last >= numel) return POTS_STORE_OTHER;
  }
  if (numel == 0 || last >= numel) return POTS_STORE_OTHER;

  memset(out, 0, sizeof *out);
  out->data_offset = at;
  out->storage_bytes = data->usize;
  out->storage_offset = (uint64_t)off;
  out->ndim = (uint32_t)size.size();
  for (size_t d = 0; d < size.size(); ++d) {
    out->size[d] = size[d].i;
    out->stride[d] = stride[d].i;
  }
  out->dtype = t.dtype;
  return POTS_STORE_OK;
}

uint32_t clamp_threads(uint32_t n) {
  return n == 0 ? kDefaultThreads : std::min(n, kMaxThreads);
}

// Run fn(0 .. n-1) on up to `threads` threads, each taking the next index.
template <class F>
void parallel_for(uint64_t n, uint32_t threads, F fn) {
  std::atomic<uint64_t> next{0};
  auto work = [&]() {
    for (uint64_t k; (k = next.fetch_add(1)) < n;) fn(k);
  };
  const uint32_t t = (uint32_t)std::min<uint64_t>(threads, n);
  std::vector<std::thread> pool;
  for (uint32_t k = 1; k < t; ++k) pool.emplace_back(work);
  work();
  for (auto& th : pool) th.join();
}

// A run of the destination, [lo, hi), that one staging slot carries: the pieces of segments
// inside it.
struct Span {
  uint64_t lo, hi;
  uint32_t first, count;  // into the piece list
};
struct Piece {
  uint32_t file;
  uint64_t file_offset, bytes, dst_offset;
};

}  // namespace
}  // namespace pots

using namespace pots;

extern "C" int pots_store_scan(uint32_t n_files, const char* const* paths,
                               pots_stored_tensor* out, uint32_t n_threads) {
  if (n_files == 0) return POTS_E_OK;
  if (!paths || !out) return POTS_E_ARG;
  for (uint32_t k = 0; k < n_files; ++k)
    if (!paths[k]) return POTS_E_ARG;
  parallel_for(n_files, clamp_threads(n_threads), [&](uint64_t k) {
    pots_stored_tensor r;
    memset(&r, 0, sizeof r);
    r.status = scan_one(paths[k], &r);
    out[k] = r;
  });
  return POTS_E_OK;
}

extern "C" int pots_store_load(uint32_t n_files, const char* const* paths, uint32_t n_segs,
                               const pots_store_segment* segs, void* dst, int dst_device,
                               void* staging, uint64_t staging_bytes, uint32_t n_threads) {
  if (n_segs == 0) return POTS_E_OK;
  if (!paths || !segs || !dst) return POTS_E_ARG;
  const uint32_t threads = clamp_threads(n_threads);
  uint64_t end = 0;
  for (uint32_t k = 0; k < n_segs; ++k) {
    const auto& s = segs[k];
    if (s.file >= n_files || !paths[s.file] || s.bytes == 0 || s.dst_offset < end ||
        s.dst_offset + s.bytes < s.dst_offset)
      return POTS_E_ARG;
    end = s.dst_offset + s.bytes;
  }
  const bool host = dst_device < 0;
  const uint64_t slot = host ? (64ull << 20)
                             : (staging_bytes / (2ull * threads)) / 4096 * 4096;
  if (!host && (!staging || slot < kMinSlot)) return POTS_E_ARG;

  // Cut the destination into spans of at most one slot; a segment longer than a slot spans
  // several.
  std::vector<Piece> pieces;
  std::vector<Span> spans;
  for (uint32_t k = 0; k < n_segs; ++k) {
    const auto& s = segs[k];
    for (uint64_t done = 0; done < s.bytes;) {
      const uint64_t d = s.dst_offset + done;
      if (spans.empty() || d + 1 > spans.back().lo + slot) {
        spans.push_back(Span{d, d, (uint32_t)pieces.size(), 0});
      }
      Span& sp = spans.back();
      const uint64_t room = sp.lo + slot - d;
      const uint64_t take = std::min(room, s.bytes - done);
      pieces.push_back(Piece{s.file, s.file_offset + done, take, d});
      sp.hi = d + take;
      ++sp.count;
      done += take;
    }
  }

  std::atomic<int> status{POTS_E_OK};
  std::string err;
  std::mutex err_mu;
  auto fail = [&](int code, const std::string& msg) {
    int ok = POTS_E_OK;
    if (status.compare_exchange_strong(ok, code)) {
      std::lock_guard<std::mutex> g(err_mu);
      err = msg;
    }
  };
  // Read one span's pieces to `base` (its byte lo lands at base[0]).
  auto read_span = [&](const Span& sp, uint8_t* base) {
    int fd = -1;
    uint32_t open_file = UINT32_MAX;
    bool ok = true;
    for (uint32_t q = sp.first; ok && q < sp.first + sp.count; ++q) {
      const Piece& pc = pieces[q];
      if (pc.file != open_file) {
        if (fd >= 0) ::close(fd);
        fd = ::open(paths[pc.file], O_RDONLY | O_CLOEXEC);
        open_file = pc.file;
        if (fd < 0) {
          fail(POTS_E_IO, std::string("cannot open ") + paths[pc.file] + ": " + strerror(errno));
          ok = false;
          break;
        }
      }
      if (!read_at(fd, base + (pc.dst_offset - sp.lo), pc.bytes, pc.file_offset)) {
        fail(POTS_E_IO, std::string("short or failed read of ") + paths[pc.file]);
        ok = false;
      }
    }
    if (fd >= 0) ::close(fd);
    return ok;
  };

  const uint64_t n_spans = spans.size();
  const uint32_t t_used = (uint32_t)std::min<uint64_t>(threads, n_spans);
  auto worker = [&](uint32_t t) {
    if (host) {
      for (uint64_t k = t; k < n_spans && status.load() == POTS_E_OK; k += t_used)
        read_span(spans[k], static_cast<uint8_t*>(dst) + spans[k].lo);
      return;
    }
    hipError_t e = hipSetDevice(dst_device);
    hipStream_t s = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    for (int b = 0; b < 2 && e == hipSuccess; ++b)
      e = hipEventCreateWithFlags(&ev[b], hipEventDisableTiming);
    uint8_t* slots = static_cast<uint8_t*>(staging) + 2ull * t * slot;
    uint32_t use = 0;
    for (uint64_t k = t; e == hipSuccess && k < n_spans && status.load() == POTS_E_OK;
         k += t_used, use ^= 1) {
      const Span& sp = spans[k];
      if (pending[use]) {
        e = hipEventSynchronize(ev[use]);
        pending[use] = false;
        if (e != hipSuccess) break;
      }
      uint8_t* buf = slots + use * slot;
      if (!read_span(sp, buf)) break;
      e = hipMemcpyAsync(static_cast<uint8_t*>(dst) + sp.lo, buf, sp.hi - sp.lo,
                         hipMemcpyHostToDevice, s);
      if (e == hipSuccess) e = hipEventRecord(ev[use], s);
      if (e == hipSuccess) pending[use] = true;
    }
    if (s) {
      const hipError_t e2 = hipStreamSynchronize(s);
      if (e == hipSuccess) e = e2;
    }
    for (auto x : ev)
      if (x) (void)hipEventDestroy(x);
    if (s) (void)hipStreamDestroy(s);
    if (e != hipSuccess)
      fail(e == hipErrorOutOfMemory ? POTS_E_NOMEM : POTS_E_HIP,
           std::string("HIP error in pots_store_load: ") + hipGetErrorString(e));
  };
  std::vector<std::thread> pool;
  for (uint32_t t = 1; t < t_used; ++t) pool.emplace_back(worker, t);
  worker(0);
  for (auto& th : pool) th.join();
  const int rc = status.load();
  if (rc != POTS_E_OK) note_error(err);
  return rc;
}
