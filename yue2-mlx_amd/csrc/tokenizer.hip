// Text side of the request, host only: the checkpoint-native tiktoken BPE
// (lyra::Tokenizer, protocol.hpp:5-16, protocol.mm:428-591) and the prompt
// layout around the AR prefixes (instruction, SongRequest::text / validate,
// token_prefixes, negative_prefix, chunk_ranges: protocol.mm:123-369).
//
// encode(text): strict UTF-8 -> code points -> NFC (the reference's
// precomposedStringWithCanonicalMapping) -> pre-tokenizer pieces -> byte
// pair merges of each piece's UTF-8 bytes. The pre-tokenizer is the
// reference's pattern
//   (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}|
//    ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+
// restated as a scanner over code points, alternatives tried in order with
// the backtracking outcome of each written out; \s is the ICU class
// [\t\n\f\r\p{Z}] (NSRegularExpression is ICU), \p{L} / \p{N} the general
// categories L* / N*. Unicode data: unicode_tables.h.
#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cstdint>
#include <cmath>
#include <cstring>
#include <fstream>
#include <iterator>
#include <queue>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "abi_util.h"
#include "common.h"
#include "unicode_tables.h"

namespace yuear {
namespace {

constexpr int kAbcStart = 151847, kMusicStart = 151851;

// ---- Unicode properties ----
template <class T, size_t N> bool in_ranges(const T (&r)[N], uint32_t cp) {
  size_t lo = 0, hi = N;
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    if (cp < r[mid].lo)
      hi = mid;
    else if (cp > r[mid].hi)
      lo = mid + 1;
    else
      return true;
  }
  return false;
}
bool is_letter(uint32_t cp) { return in_ranges(unicode::kLetters, cp); }
bool is_number(uint32_t cp) { return in_ranges(unicode::kNumbers, cp); }
bool is_space(uint32_t cp) {  // ICU \s
  return cp == '\t' || cp == '\n' || cp == '\f' || cp == '\r' ||
         in_ranges(unicode::kSeparators, cp);
}
bool is_crlf(uint32_t cp) { return cp == '\r' || cp == '\n'; }

uint32_t combining_class(uint32_t cp) {
  const auto &t = unicode::kCombining;
  size_t lo = 0, hi = std::size(t);
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    if (cp < t[mid].lo)
      hi = mid;
    else if (cp > t[mid].hi)
      lo = mid + 1;
    else
      return t[mid].ccc;
  }
  return 0;
}

// ---- UTF-8 ----
// Strict decoding (RFC 3629: no overlong forms, no surrogates, <= U+10FFFF).
std::vector<uint32_t> utf8_decode(std::string_view s) {
  std::vector<uint32_t> out;
  out.reserve(s.size());
  auto bad = [] { throw Error("UnicodeDecodeError", "Invalid UTF-8 text"); };
  for (size_t i = 0; i < s.size();) {
    const uint32_t c = static_cast<unsigned char>(s[i]);
    if (c < 0x80) {
      out.push_back(c);
      ++i;
      continue;
    }
    int n = 0;
    uint32_t cp = 0, min = 0;
    if (c >= 0xC2 && c <= 0xDF)
      n = 2, cp = c & 0x1F, min = 0x80;
    else if (c >= 0xE0 && c <= 0xEF)
      n = 3, cp = c & 0x0F, min = 0x800;
    else if (c >= 0xF0 && c <= 0xF4)
      n = 4, cp = c & 0x07, min = 0x10000;
    else
      bad();
    if (i + n > s.size())
      bad();
    for (int k = 1; k < n; ++k) {
      const uint32_t d = static_cast<unsigned char>(s[i + k]);
      if ((d & 0xC0) != 0x80)
        bad();
      cp = (cp << 6) | (d & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))
      bad();
    out.push_back(cp);
    i += n;
  }
  return out;
}
void utf8_append(std::string &out, uint32_t cp) {
  if (cp < 0x80) {
    out += char(cp);
  } else if (cp < 0x800) {
    out += char(0xC0 | (cp >> 6));
    out += char(0x80 | (cp & 0x3F));
  } else if (cp < 0x10000) {
    out += char(0xE0 | (cp >> 12));
    out += char(0x80 | ((cp >> 6) & 0x3F));
    out += char(0x80 | (cp & 0x3F));
  } else {
    out += char(0xF0 | (cp >> 18));
    out += char(0x80 | ((cp >> 12) & 0x3F));
    out += char(0x80 | ((cp >> 6) & 0x3F));
    out += char(0x80 | (cp & 0x3F));
  }
}

// Invalid UTF-8 -> U+FFFD per maximal subpart, as Python's
// bytes.decode(errors="replace") (protocol.mm:86-114).
std::string replacement_utf8(std::string_view s) {
  std::string out;
  out.reserve(s.size());
  for (size_t i = 0; i < s.size();) {
    const unsigned c = static_cast<unsigned char>(s[i]);
    if (c < 0x80) {
      out += s[i++];
      continue;
    }
    const int n = c >= 0xC2 && c <= 0xDF ? 2 : c >= 0xE0 && c <= 0xEF ? 3
                                            : c >= 0xF0 && c <= 0xF4 ? 4 : 0;
    // second-byte bounds that exclude overlong forms, surrogates and > U+10FFFF
    const unsigned lo = c == 0xE0 ? 0xA0 : c == 0xF0 ? 0x90 : 0x80;
    const unsigned hi = c == 0xED ? 0x9F : c == 0xF4 ? 0x8F : 0xBF;
    size_t len = 1;
    while (n && len < size_t(n) && i + len < s.size()) {
      const unsigned d = static_cast<unsigned char>(s[i + len]);
      if (d < (len == 1 ? lo : 0x80) || d > (len == 1 ? hi : 0xBF))
        break;
      ++len;
    }
    if (n && len == size_t(n))
      out.append(s.substr(i, len));
    else
      out += "\xEF\xBF\xBD";
    i += len;
  }
  return out;
}

// ---- NFC (UAX #15: full canonical decomposition, canonical ordering,
// canonical composition; Hangul arithmetically) ----
constexpr uint32_t kSBase = 0xAC00, kLBase = 0x1100, kVBase = 0x1161, kTBase = 0x11A7;
constexpr uint32_t kLCount = 19, kVCount = 21, kTCount = 28, kNCount = kVCount * kTCount,
                   kSCount = kLCount * kNCount;

void decompose(uint32_t cp, std::vector<uint32_t> &out) {
  if (cp >= kSBase && cp < kSBase + kSCount) {
    const uint32_t s = cp - kSBase;
    out.push_back(kLBase + s / kNCount);
    out.push_back(kVBase + (s % kNCount) / kTCount);
    if (s % kTCount)
      out.push_back(kTBase + s % kTCount);
    return;
  }
  const auto &t = unicode::kDecompositions;
  const auto it = std::lower_bound(std::begin(t), std::end(t), cp,
                                   [](const unicode::Decomposition &d, uint32_t v) {
                                     return d.cp < v;
                                   });
  if (it == std::end(t) || it->cp != cp) {
    out.push_back(cp);
    return;
  }
  decompose(it->first, out);
  if (it->second)
    decompose(it->second, out);
}

// Primary composite of (a, b), or 0.
uint32_t compose(uint32_t a, uint32_t b) {
  if (a >= kLBase && a < kLBase + kLCount && b >= kVBase && b < kVBase + kVCount)
    return kSBase + ((a - kLBase) * kVCount + (b - kVBase)) * kTCount;
  if (a >= kSBase && a < kSBase + kSCount && (a - kSBase) % kTCount == 0 && b > kTBase &&
      b < kTBase + kTCount)
    return a + (b - kTBase);
  const auto &t = unicode::kComposites;
  const auto it = std::lower_bound(std::begin(t), std::end(t), std::pair<uint32_t, uint32_t>(a, b),
                                   [](const unicode::Composite &c, std::pair<uint32_t, uint32_t> v) {
                                     return c.first != v.first ? c.first < v.first
                                                               : c.second < v.second;
                                   });
  return it != std::end(t) && it->first == a && it->second == b ? it->cp : 0;
}

std::vector<uint32_t> nfc(const std::vector<uint32_t> &in) {
  std::vector<uint32_t> d;
  d.reserve(in.size() + in.size() / 4);
  for (uint32_t cp : in)
    decompose(cp, d);
  std::vector<uint32_t> cc(d.size());
  for (size_t i = 0; i < d.size(); ++i)
    cc[i] = combining_class(d[i]);
  // canonical ordering: stable sort of each run of non-starters by class
  for (size_t i = 0; i < d.size();) {
    if (!cc[i]) {
      ++i;
      continue;
    }
    size_t j = i;
    while (j < d.size() && cc[j])
      ++j;
    for (size_t a = i + 1; a < j; ++a)  // insertion sort (runs are short)
      for (size_t b = a; b > i && cc[b - 1] > cc[b]; --b) {
        std::swap(d[b - 1], d[b]);
        std::swap(cc[b - 1], cc[b]);
      }
    i = j;
  }
  // composition: c joins the last starter unless a character between them
  // has class 0 or a class >= c's (blocked); the non-starters kept after the
  // starter are in non-decreasing class order, so the last one decides
  std::vector<uint32_t> out;
  out.reserve(d.size());
  size_t starter = SIZE_MAX;
  uint32_t last_cc = 0;
  for (size_t i = 0; i < d.size(); ++i) {
    const uint32_t c = d[i], k = cc[i];
    if (starter != SIZE_MAX) {
      const bool adjacent = out.size() == starter + 1;
      if (adjacent || (k && last_cc < k)) {
        const uint32_t p = compose(out[starter], c);
        if (p) {
          out[starter] = p;
          continue;
        }
      }
    }
    if (!k) {
      starter = out.size();
      last_cc = 0;
    } else {
      last_cc = k;
    }
    out.push_back(c);
  }
  return out;
}

// ---- pre-tokenizer: end of the piece starting at i ----
uint32_t fold_ascii(uint32_t c) {
  if (c == 0x17F)  // LATIN SMALL LETTER LONG S case-folds to 's'
    return 's';
  return c >= 'A' && c <= 'Z' ? c + 32 : c;
}
size_t piece_end(const std::vector<uint32_t> &c, size_t i) {
  const size_t n = c.size();
  // (?i:'s|'t|'re|'ve|'m|'ll|'d)
  if (c[i] == '\'' && i + 1 < n) {
    const uint32_t x = fold_ascii(c[i + 1]);
    if (x == 's' || x == 't' || x == 'm' || x == 'd')
      return i + 2;
    if (i + 2 < n) {
      const uint32_t y = fold_ascii(c[i + 2]);
      if ((x == 'r' && y == 'e') || (x == 'v' && y == 'e') || (x == 'l' && y == 'l'))
        return i + 3;
    }
  }
  // [^\r\n\p{L}\p{N}]?\p{L}+
  size_t j = i;
  if (!is_letter(c[j]) && !is_crlf(c[j]) && !is_number(c[j]) && j + 1 < n && is_letter(c[j + 1]))
    ++j;
  if (is_letter(c[j])) {
    while (j < n && is_letter(c[j]))
      ++j;
    return j;
  }
  // \p{N}
  if (is_number(c[i]))
    return i + 1;
  //  ?[^\s\p{L}\p{N}]+[\r\n]*
  auto other = [&](uint32_t x) { return !is_space(x) && !is_letter(x) && !is_number(x); };
  j = i + (c[i] == ' ' && i + 1 < n && other(c[i + 1]) ? 1 : 0);
  if (other(c[j])) {
    while (j < n && other(c[j]))
      ++j;
    while (j < n && is_crlf(c[j]))
      ++j;
    return j;
  }
  // c[i] is whitespace here. \s*[\r\n]+: up to the last CR/LF of the run
  size_t e = i, last = SIZE_MAX;
  for (; e < n && is_space(c[e]); ++e)
    if (is_crlf(c[e]))
      last = e;
  if (last != SIZE_MAX)
    return last + 1;
  // \s+(?!\S): the run, less its last character when a non-space follows
  if (e == n || e - i >= 2)
    return e == n ? e : e - 1;
  return e;  // \s+
}

// NSCharacterSet whitespaceAndNewlineCharacterSet (Z*, U+0009-000D, U+0085)
// plus U+001C-001F (protocol.mm:71-80).
bool nonwhite(std::string_view s) {
  for (uint32_t cp : utf8_decode(s)) {
    const bool white = (cp >= 0x09 && cp <= 0x0D) || cp == 0x85 || (cp >= 0x1C && cp <= 0x1F) ||
                       in_ranges(unicode::kSeparators, cp);
    if (!white)
      return true;
  }
  return false;
}

// ---- base64 (RFC 4648, padded) ----
bool base64_decode(std::string_view in, std::string &out) {
  auto value = [](char ch) -> int {
    if (ch >= 'A' && ch <= 'Z') return ch - 'A';
    if (ch >= 'a' && ch <= 'z') return ch - 'a' + 26;
    if (ch >= '0' && ch <= '9') return ch - '0' + 52;
    if (ch == '+') return 62;
    if (ch == '/') return 63;
    return -1;
  };
  out.clear();
  if (in.empty() || in.size() % 4)
    return false;
  for (size_t i = 0; i < in.size(); i += 4) {
    const bool tail = i + 4 == in.size();
    int v[4];
    int pad = 0;
    for (int k = 0; k < 4; ++k) {
      if (in[i + k] == '=' && tail && k >= 2) {
        v[k] = 0;
        ++pad;
        continue;
      }
      if (pad || (v[k] = value(in[i + k])) < 0)
        return false;
    }
    const uint32_t w = (uint32_t(v[0]) << 18) | (uint32_t(v[1]) << 12) | (uint32_t(v[2]) << 6) |
                       uint32_t(v[3]);
    out += char(w >> 16);
    if (pad < 2)
      out += char((w >> 8) & 0xFF);
    if (pad < 1)
      out += char(w & 0xFF);
  }
  return true;
}

}  // namespace

// lyra::Tokenizer (protocol.mm:428-591).
struct TextTokenizer {
  std::unordered_map<std::string, int> ranks;
  std::vector<std::string> pieces;

  explicit TextTokenizer(const std::string &path) : pieces(kEOD + 208) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
      const int e = errno;
      throw Error(e == ENOENT ? "FileNotFoundError"
                  : e == EACCES || e == EPERM ? "PermissionError" : "OSError",
                  path + ": " + std::strerror(e));
    }
    const std::string text((std::istreambuf_iterator<char>(f)), {});
    ranks.reserve(kEOD);
    std::string piece;
    for (size_t at = 0; at < text.size();) {
      size_t end = text.find('\n', at);
      if (end == std::string::npos)
        end = text.size();
      const std::string_view line(text.data() + at, end - at);
      at = end + 1;
      if (line.empty())
        continue;
      // two whitespace-separated fields: base64 piece, rank in [0, EOD)
      std::vector<std::string_view> fields;
      for (size_t p = 0; p < line.size();) {
        while (p < line.size() && std::isspace(static_cast<unsigned char>(line[p])))
          ++p;
        size_t q = p;
        while (q < line.size() && !std::isspace(static_cast<unsigned char>(line[q])))
          ++q;
        if (q > p)
          fields.push_back(line.substr(p, q - p));
        p = q;
      }
      // the rank reads as a C++ stream int: optional sign, digits, no overflow
      long long rank = 0;
      bool ok = fields.size() == 2;
      if (ok) {
        const std::string_view r = fields[1];
        const bool neg = r[0] == '-';
        size_t k = r[0] == '+' || neg ? 1 : 0;
        ok = k < r.size();
        for (; ok && k < r.size(); ++k) {
          ok = std::isdigit(static_cast<unsigned char>(r[k])) && rank <= (1LL << 31);
          rank = rank * 10 + (r[k] - '0');
        }
        ok = ok && rank <= (neg ? (1LL << 31) : (1LL << 31) - 1);
        if (neg)
          rank = -rank;
      }
      if (!ok || rank < 0 || rank >= kEOD)
        invalid("Invalid checkpoint-native qwen.tiktoken vocabulary");
      if (!base64_decode(fields[0], piece) || piece.empty())
        invalid("Invalid base64 vocabulary token");
      ranks[piece] = int(rank);
      pieces[size_t(rank)] = piece;
    }
    if (ranks.size() != size_t(kEOD) ||
        std::any_of(pieces.begin(), pieces.begin() + kEOD, [](const auto &s) { return s.empty(); }))
      invalid("Expected checkpoint-native qwen.tiktoken (151643 ordinary tokens)");
    const char *specials[] = {"<|endoftext|>", "<|im_start|>", "<|im_end|>", "<R>",
                              "<S>",           "<X>",          "<mask>",     "<sep>"};
    for (int i = 0; i < 8; ++i)
      pieces[size_t(kEOD + i)] = specials[i];
    for (int i = 0; i < 200; ++i)
      pieces[size_t(kEOD + 8 + i)] = "<extra_" + std::to_string(i) + ">";
    pieces[kAbcStart] = "<abc>";
    pieces[kAbcEnd] = "</abc>";
  }

  int rank_of(std::string_view s) const {
    const auto it = ranks.find(std::string(s));
    return it == ranks.end() ? -1 : it->second;
  }

  // Byte pair merges of one piece: repeatedly join the adjacent pair whose
  // concatenation has the lowest rank (leftmost on ties) until no
  // concatenation is in the vocabulary; a piece that is itself in the
  // vocabulary is one token.
  void bpe(std::string_view w, std::vector<int32_t> &out) const {
    const int direct = rank_of(w);
    if (direct >= 0) {
      out.push_back(direct);
      return;
    }
    const int n = int(w.size());
    std::vector<int> next(n), prev(n), end(n), stamp(n, 0);
    for (int i = 0; i < n; ++i) {
      next[i] = i + 1 < n ? i + 1 : -1;
      prev[i] = i - 1;
      end[i] = i + 1;
    }
    struct Cand {
      int rank, left, stamp_l, stamp_r;
      bool operator<(const Cand &o) const {  // max-heap: lowest rank, then leftmost, on top
        return rank != o.rank ? rank > o.rank : left > o.left;
      }
    };
    std::priority_queue<Cand> heap;
    auto push = [&](int l) {
      if (l < 0 || next[l] < 0)
        return;
      const int r = next[l];
      const int rk = rank_of(w.substr(size_t(l), size_t(end[r] - l)));
      if (rk >= 0)
        heap.push({rk, l, stamp[l], stamp[r]});
    };
    for (int i = 0; i + 1 < n; ++i)
      push(i);
    while (!heap.empty()) {
      const Cand c = heap.top();
      heap.pop();
      const int l = c.left, r = next[l];
      if (r < 0 || stamp[l] != c.stamp_l || stamp[r] != c.stamp_r || stamp[l] < 0)
        continue;  // stale: one side changed since the candidate was made
      end[l] = end[r];
      next[l] = next[r];
      if (next[r] >= 0)
        prev[next[r]] = l;
      stamp[r] = -1;  // r is gone
      ++stamp[l];
      push(prev[l]);
      push(l);
    }
    for (int i = 0; i >= 0; i = next[i]) {
      const int rk = rank_of(w.substr(size_t(i), size_t(end[i] - i)));
      if (rk < 0)
        invalid("Vocabulary is missing a byte token");
      out.push_back(rk);
    }
  }

  std::vector<int32_t> encode(std::string_view text) const {
    const std::vector<uint32_t> cps = nfc(utf8_decode(text));
    std::vector<int32_t> out;
    std::string bytes;
    for (size_t i = 0; i < cps.size();) {
      const size_t j = piece_end(cps, i);
      bytes.clear();
      for (size_t k = i; k < j; ++k)
        utf8_append(bytes, cps[k]);
      bpe(bytes, out);
      i = j;
    }
    return out;
  }

  std::string decode(const int32_t *ids, size_t n) const {
    std::string raw;
    for (size_t i = 0; i < n; ++i)
      if (ids[i] >= 0 && size_t(ids[i]) < pieces.size())
        raw += pieces[size_t(ids[i])];
    return replacement_utf8(raw);
  }
};

namespace {

// instruction (protocol.mm:200-211)
std::string instruction(const char *cot) {
  const std::string c = cot ? cot : "";
  if (c == "off")
    return "Generate music with codec tokens from the given conditions.";
  if (c == "melody")
    return "Generate a melody-only ABC transcription without chord symbols, then generate "
           "music with codec tokens from the given conditions.";
  if (c == "full")
    return "Generate a chord-annotated ABC transcription, then generate music with codec "
           "tokens from the given conditions.";
  invalid("cot must be off, melody or full");
}

// SongRequest::text (protocol.mm:242-245)
std::string request_text(const yuear_song_request &r) {
  return instruction(r.cot) + "\n[Tags]\n" + std::string(r.style ? r.style : "") +
         "\n[Lyrics]\n" + std::string(r.lyrics ? r.lyrics : "") + "\n";
}

void abc_valid(const int32_t *ids, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= kEOD)
      invalid("ABC IDs must remain inside the ordinary text vocabulary");
}

void give_ids(const std::vector<int32_t> &v, int32_t **ids, int64_t *n) {
  if (!ids || !n)
    invalid("ids and n must not be NULL");
  *ids = static_cast<int32_t *>(std::malloc(std::max<size_t>(1, v.size()) * sizeof(int32_t)));
  if (!*ids)
    throw Error("MemoryError", "out of host memory");
  std::copy(v.begin(), v.end(), *ids);
  *n = int64_t(v.size());
}

void check_request(const yuear_song_request *r) {
  if (!r || !r->style || !r->lyrics)
    invalid("Provide style and lyrics");
}

}  // namespace
}  // namespace yuear

using yuear::TextTokenizer;

struct yuear_tokenizer {
  TextTokenizer impl;
  explicit yuear_tokenizer(const std::string &p) : impl(p) {}
};

extern "C" {

yuear_status yuear_tokenizer_load(const char *vocabulary, yuear_tokenizer **out,
                                  char **error_json) {
  return yuear::guarded(error_json, [&] {
    if (!vocabulary || !out)
      yuear::invalid("vocabulary and out must not be NULL");
    *out = nullptr;
    *out = new yuear_tokenizer(vocabulary);
  });
}

void yuear_tokenizer_destroy(yuear_tokenizer *t) { delete t; }

void yuear_ids_free(int32_t *ids) { std::free(ids); }

yuear_status yuear_tokenizer_encode(const yuear_tokenizer *t, const char *text, int64_t len,
                                    int32_t **ids, int64_t *n, char **error_json) {
  return yuear::guarded(error_json, [&] {
    if (!t || (!text && len) || len < 0)
      yuear::invalid("tokenizer and text must not be NULL");
    yuear::give_ids(t->impl.encode(std::string_view(text ? text : "", size_t(len))), ids, n);
  });
}

yuear_status yuear_tokenizer_decode(const yuear_tokenizer *t, const int32_t *ids, int64_t n,
                                    char **text, int64_t *len, char **error_json) {
  return yuear::guarded(error_json, [&] {
    if (!t || (!ids && n) || n < 0 || !text)
      yuear::invalid("tokenizer, ids and text must not be NULL");
    const std::string s = t->impl.decode(ids, size_t(n));
    *text = static_cast<char *>(std::malloc(s.size() + 1));
    if (!*text)
      throw yuear::Error("MemoryError", "out of host memory");
    std::memcpy(*text, s.data(), s.size());
    (*text)[s.size()] = 0;
    if (len)
      *len = int64_t(s.size());
  });
}

yuear_status yuear_text_nfc(const char *text, int64_t len, char **out, int64_t *out_len,
                            char **error_json) {
  return yuear::guarded(error_json, [&] {
    if ((!text && len) || len < 0 || !out)
      yuear::invalid("text and out must not be NULL");
    std::string s;
    for (uint32_t cp : yuear::nfc(yuear::utf8_decode(std::string_view(text ? text : "", size_t(len)))))
      yuear::utf8_append(s, cp);
    *out = static_cast<char *>(std::malloc(s.size() + 1));
    if (!*out)
      throw yuear::Error("MemoryError", "out of host memory");
    std::memcpy(*out, s.data(), s.size());
    (*out)[s.size()] = 0;
    if (out_len)
      *out_len = int64_t(s.size());
  });
}

yuear_status yuear_text_pieces(const char *text, int64_t len, int32_t **ends, int64_t *n,
                               char **error_json) {
  return yuear::guarded(error_json, [&] {
    if ((!text && len) || len < 0)
      yuear::invalid("text must not be NULL");
    const std::vector<uint32_t> cps =
        yuear::nfc(yuear::utf8_decode(std::string_view(text ? text : "", size_t(len))));
    std::vector<int32_t> out;
    std::string bytes;
    for (size_t i = 0; i < cps.size();) {
      const size_t j = yuear::piece_end(cps, i);
      for (size_t k = i; k < j; ++k)
        yuear::utf8_append(bytes, cps[k]);
      out.push_back(int32_t(bytes.size()));
      i = j;
    }
    yuear::give_ids(out, ends, n);
  });
}

yuear_status yuear_song_request_validate(const yuear_song_request *r, char **error_json) {
  return yuear::guarded(error_json, [&] {
    yuear::check_request(r);
    yuear::instruction(r->cot);
    if (r->seed >= (uint64_t(1) << 63))
      yuear::invalid("seed must be an integer in [0, 2**63)");
    const std::string id = r->id ? r->id : "";
    auto alnum = [](unsigned char c) {
      return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9');
    };
    if (id.empty() || id.size() > 180 || !alnum(id[0]) ||
        !std::all_of(id.begin(), id.end(), [&](unsigned char c) {
          return alnum(c) || c == '_' || c == '.' || c == '-';
        }))
      yuear::invalid("id must be a filename-safe identifier");
    if (r->abc && (std::string(r->cot) == "off" || !yuear::nonwhite(r->abc)))
      yuear::invalid("External ABC requires nonempty text and cot=melody/full");
    if (r->has_cfg_scale && (!std::isfinite(r->cfg_scale) || r->cfg_scale < 0 || r->cfg_scale > 20))
      yuear::invalid("cfg_scale must be finite and in [0,20]");
  });
}

double yuear_song_request_guidance(const yuear_song_request *r) {
  if (!r)
    return 1.;
  if (r->has_cfg_scale)
    return r->cfg_scale;
  return r->cot && std::string(r->cot) == "off" ? 1.01 : 1.;
}

yuear_status yuear_token_prefixes(const yuear_tokenizer *t, const yuear_song_request *r,
                                  const int32_t *abc_ids, int64_t n_abc, int32_t has_abc_ids,
                                  int32_t **ids, int64_t *n, char **error_json) {
  return yuear::guarded(error_json, [&] {
    yuear::check_request(r);
    if (!t || (has_abc_ids && n_abc && !abc_ids) || n_abc < 0)
      yuear::invalid("tokenizer and abc_ids must not be NULL");
    const std::string text = yuear::request_text(*r);
    std::vector<int32_t> out{yuear::kEOD};
    const auto body = t->impl.encode(text);
    out.insert(out.end(), body.begin(), body.end());
    out.push_back(yuear::kAbcStart);
    if (std::string(r->cot) == "off") {
      out.insert(out.end(), {yuear::kAbcEnd, yuear::kMusicStart});
    } else if (has_abc_ids || r->abc) {
      std::vector<int32_t> abc;
      if (has_abc_ids)
        abc.assign(abc_ids, abc_ids + n_abc);
      else
        abc = t->impl.encode(r->abc);
      yuear::abc_valid(abc.data(), int64_t(abc.size()));
      out.insert(out.end(), abc.begin(), abc.end());
      out.insert(out.end(), {yuear::kAbcEnd, yuear::kMusicStart});
    }
    yuear::give_ids(out, ids, n);
  });
}

yuear_status yuear_negative_prefix(const yuear_tokenizer *t, const yuear_song_request *r,
                                   const int32_t *abc_ids, int64_t n_abc, int32_t has_abc_ids,
                                   int32_t **ids, int64_t *n, char **error_json) {
  return yuear::guarded(error_json, [&] {
    yuear::check_request(r);
    if (!t || (has_abc_ids && n_abc && !abc_ids) || n_abc < 0)
      yuear::invalid("tokenizer and abc_ids must not be NULL");
    std::vector<int32_t> out{yuear::kEOD};
    const auto body = t->impl.encode(yuear::instruction(r->cot));
    out.insert(out.end(), body.begin(), body.end());
    if (std::string(r->cot) == "off") {
      out.push_back(yuear::kMusicStart);
    } else {
      if (!has_abc_ids)
        yuear::invalid("Symbolic CFG must retain the exact positive-branch ABC IDs");
      yuear::abc_valid(abc_ids, n_abc);
      out.push_back(yuear::kAbcStart);
      out.insert(out.end(), abc_ids, abc_ids + n_abc);
      out.insert(out.end(), {yuear::kAbcEnd, yuear::kMusicStart});
    }
    yuear::give_ids(out, ids, n);
  });
}

yuear_status yuear_chunk_ranges(int32_t frames, int32_t prefix_tokens, int32_t context,
                                int32_t **bounds, int64_t *n, char **error_json) {
  return yuear::guarded(error_json, [&] {
    const int64_t available = int64_t(context) - prefix_tokens - 3;
    if (frames < 1 || available < 2)
      yuear::invalid("Empty codec or prefix leaves no acoustic context");
    const int64_t size = std::min<int64_t>(available / 2, yuear::kContext);
    std::vector<int32_t> out;
    out.reserve(size_t((int64_t(frames) + size - 1) / size) * 2);
    for (int64_t a = 0; a < frames; a += size) {
      out.push_back(int32_t(a));
      out.push_back(int32_t(std::min<int64_t>(a + size, frames)));
    }
    yuear::give_ids(out, bounds, n);
    *n /= 2;
  });
}

}  // extern "C"
