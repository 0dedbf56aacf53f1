// WordPiece tokenizer (io/tokenizer.zig) on the host, behind the C ABI.
//
// Byte-level, as the reference: whitespace is ' ', '\t', '\n', '\r'
// (tokenizer.zig:267-269), punctuation the ASCII set of tokenizer.zig:271-276,
// lowercasing ASCII only (278-284), words longer than 200 bytes become [UNK]
// (tokenizer.zig:163-166, 215-218), and the longest-prefix search tries
// every shorter end before giving the whole word [UNK] (tokenizer.zig:177-206,
// 229-259).  The vocabulary is an open-addressing table over one byte arena,
// so a lookup of a candidate piece allocates nothing.
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "common.h"

namespace {

bool is_space(uint8_t c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r'; }

bool is_punct(uint8_t c) {
    // ! " # $ % & ' ( ) * + , - . / : ; < = > ? @ [ \ ] ^ _ ` { | } ~
    return (c >= 33 && c <= 47) || (c >= 58 && c <= 64) || (c >= 91 && c <= 96) || (c >= 123 && c <= 126);
}

uint64_t hash_bytes(const uint8_t *p, size_t n) {
    uint64_t h = 1469598103934665603ull;  // FNV-1a
    for (size_t i = 0; i < n; i++) h = (h ^ p[i]) * 1099511628211ull;
    return h ^ (h >> 29);
}

}  // namespace

struct tzh_tokenizer {
    uint32_t unk_id = 100, cls_id = 101, sep_id = 102;  // tokenizer.zig:12-14
    size_t max_word_chars = 200;                        // tokenizer.zig:15

    struct Slot {
        uint32_t off = 0, len = 0, id = 0;
        bool used = false;
    };
    std::string arena;
    std::vector<Slot> slots = std::vector<Slot>(1024);
    size_t count = 0;

    const Slot *find(const uint8_t *p, size_t n) const {
        const size_t mask = slots.size() - 1;
        for (size_t i = hash_bytes(p, n) & mask;; i = (i + 1) & mask) {
            const Slot &s = slots[i];
            if (!s.used) return nullptr;
            if (s.len == n && std::memcmp(arena.data() + s.off, p, n) == 0) return &s;
        }
    }

    // StringHashMap.put: a key already present takes the new value.
    void put(const uint8_t *p, size_t n, uint32_t id) {
        if ((count + 1) * 2 > slots.size()) grow();
        const size_t mask = slots.size() - 1;
        for (size_t i = hash_bytes(p, n) & mask;; i = (i + 1) & mask) {
            Slot &s = slots[i];
            if (!s.used) {
                s.off = (uint32_t)arena.size();
                s.len = (uint32_t)n;
                s.id = id;
                s.used = true;
                arena.append((const char *)p, n);
                count++;
                return;
            }
            if (s.len == n && std::memcmp(arena.data() + s.off, p, n) == 0) {
                s.id = id;
                return;
            }
        }
    }

    void grow() {
        std::vector<Slot> old(slots.size() * 2);
        old.swap(slots);
        const size_t mask = slots.size() - 1;
        for (const Slot &s : old) {
            if (!s.used) continue;
            size_t i = hash_bytes((const uint8_t *)arena.data() + s.off, s.len) & mask;
            while (slots[i].used) i = (i + 1) & mask;
            slots[i] = s;
        }
    }

    uint32_t get_or_unk(const uint8_t *p, size_t n) const {
        const Slot *s = find(p, n);
        return s ? s->id : unk_id;
    }

    // loadVocabFromBytes (tokenizer.zig:54-74): the id of a token is its
    // line index; empty lines count; one trailing '\r' is stripped.
    void load_bytes(const uint8_t *data, size_t len) {
        uint32_t line_idx = 0;
        size_t start = 0;
        for (;;) {
            size_t end = start;
            while (end < len && data[end] != '\n') end++;
            size_t n = end - start;
            if (n > 0 && data[start + n - 1] == '\r') n--;
            if (n > 0) put(data + start, n, line_idx);
            line_idx++;
            if (end >= len) break;
            start = end + 1;
        }
    }

    // WordPiece of one word (tokenizer.zig:154-206 and 209-259).  emit(id)
    // appends a piece and returns false when there is no room for it; a
    // word with a piece missing from the vocabulary becomes one [UNK]
    // (rewind() drops the pieces already emitted for it).
    template <typename Room, typename Emit, typename Rewind>
    void word(const uint8_t *w, size_t n, Room room, Emit emit, Rewind rewind) const {
        if (n > max_word_chars) {
            emit(unk_id);
            return;
        }
        // buf = two spare bytes + the lowercased word.  For a piece after
        // the first, the two bytes before it (already consumed) are
        // overwritten with "##", so every candidate is a prefix of
        // buf + start and no lookup copies bytes.
        uint8_t buf[2 + 256];
        for (size_t i = 0; i < n; i++) buf[2 + i] = (w[i] >= 'A' && w[i] <= 'Z') ? w[i] + 32 : w[i];
        size_t start = 0;
        bool first = true;
        while (start < n && room()) {
            const uint8_t *base = buf + 2 + start;
            size_t extra = 0;
            if (!first) {
                buf[start] = buf[start + 1] = '#';
                base -= 2;
                extra = 2;
            }
            const Slot *hit = nullptr;
            size_t end = n;
            for (; end > start; end--)
                if ((hit = find(base, end - start + extra))) break;
            if (!hit) {
                rewind();
                emit(unk_id);
                return;
            }
            emit(hit->id);
            start = end;
            first = false;
        }
    }
};

// Tokenizer.encode (tokenizer.zig:78-118): [CLS] pieces [SEP] into
// out[0, cap), cap >= 2; the text is cut where the pieces reach cap - 1
// (inside a word too), and [SEP] always ends the output.
size_t tzh_tokenize(const tzh_tokenizer *tok, const uint8_t *t, size_t len, uint32_t *out, size_t cap) {
    size_t pos = 0, i = 0;
    out[pos++] = tok->cls_id;
    while (i < len && pos < cap - 1) {
        while (i < len && is_space(t[i])) i++;
        if (i >= len) break;
        const size_t ws = i;
        while (i < len && !is_space(t[i]) && !is_punct(t[i])) i++;
        if (i > ws) {
            const size_t start_pos = pos;
            tok->word(
                t + ws, i - ws, [&] { return pos < cap - 1; }, [&](uint32_t id) { out[pos++] = id; },
                [&] { pos = start_pos; });
        }
        if (i < len && is_punct(t[i])) {
            if (pos < cap - 1) out[pos++] = tok->get_or_unk(t + i, 1);
            i++;
        }
    }
    out[pos++] = tok->sep_id;
    return pos;
}

// Tokenizer.encodeRaw (tokenizer.zig:122-151): the pieces of the whole
// text, no markers, no length limit.
void tzh_tokenize_raw(const tzh_tokenizer *tok, const uint8_t *t, size_t len, std::vector<uint32_t> &out) {
    size_t i = 0;
    while (i < len) {
        while (i < len && is_space(t[i])) i++;
        if (i >= len) break;
        const size_t ws = i;
        while (i < len && !is_space(t[i]) && !is_punct(t[i])) i++;
        if (i > ws) {
            const size_t start_len = out.size();
            tok->word(
                t + ws, i - ws, [] { return true; }, [&](uint32_t id) { out.push_back(id); },
                [&] { out.resize(start_len); });
        }
        if (i < len && is_punct(t[i])) {
            out.push_back(tok->get_or_unk(t + i, 1));
            i++;
        }
    }
}

uint32_t tzh_tokenizer_cls(const tzh_tokenizer *tok) { return tok->cls_id; }
uint32_t tzh_tokenizer_sep(const tzh_tokenizer *tok) { return tok->sep_id; }

extern "C" int tzh_tokenizer_create(tzh_tokenizer **out) {
    tzh_clear_error();
    if (!out) return tzh_fail(TZH_ERR_INVALID_ARGS, "null output handle");
    try {
        *out = new tzh_tokenizer();
    } catch (const std::bad_alloc &) {
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "tokenizer allocation failed");
    }
    return TZH_OK;
}

extern "C" int tzh_tokenizer_free(tzh_tokenizer *tok) {
    delete tok;
    return TZH_OK;
}

extern "C" int tzh_tokenizer_load_vocab_bytes(tzh_tokenizer *tok, const char *data, int64_t len) {
    tzh_clear_error();
    if (!tok || len < 0 || (!data && len > 0)) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad vocabulary arguments");
    try {
        tok->load_bytes((const uint8_t *)data, (size_t)len);
    } catch (const std::bad_alloc &) {
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "vocabulary allocation failed");
    }
    return TZH_OK;
}

extern "C" int tzh_tokenizer_load_vocab(tzh_tokenizer *tok, const char *path) {
    tzh_clear_error();
    if (!tok || !path) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad vocabulary arguments");
    std::ifstream f(path, std::ios::binary);
    if (!f) return tzh_fail(TZH_ERR_IO, "cannot open %s", path);
    std::string data((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    if (f.bad()) return tzh_fail(TZH_ERR_IO, "read of %s failed", path);
    return tzh_tokenizer_load_vocab_bytes(tok, data.data(), (int64_t)data.size());
}

extern "C" int tzh_tokenizer_put(tzh_tokenizer *tok, const char *token, int64_t len, uint32_t id) {
    tzh_clear_error();
    if (!tok || !token || len < 0 || len > 0xFFFFFF) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad token arguments");
    try {
        tok->put((const uint8_t *)token, (size_t)len, id);
    } catch (const std::bad_alloc &) {
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "vocabulary allocation failed");
    }
    return TZH_OK;
}

extern "C" int tzh_tokenizer_encode(const tzh_tokenizer *tok, const char *text, int64_t len, uint32_t *out,
                                    int64_t capacity, int64_t *n) {
    tzh_clear_error();
    if (!tok || !out || !n || len < 0 || (!text && len > 0))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "bad encode arguments");
    if (capacity < 2) return tzh_fail(TZH_ERR_INVALID_ARGS, "capacity %lld < 2 (room for [CLS] and [SEP])",
                                      (long long)capacity);
    *n = (int64_t)tzh_tokenize(tok, (const uint8_t *)text, (size_t)len, out, (size_t)capacity);
    return TZH_OK;
}

extern "C" int tzh_tokenizer_encode_raw(const tzh_tokenizer *tok, const char *text, int64_t len, uint32_t *out,
                                        int64_t capacity, int64_t *n) {
    tzh_clear_error();
    if (!tok || !n || len < 0 || capacity < 0 || (!text && len > 0) || (!out && capacity > 0))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "bad encode arguments");
    std::vector<uint32_t> ids;
    try {
        tzh_tokenize_raw(tok, (const uint8_t *)text, (size_t)len, ids);
    } catch (const std::bad_alloc &) {
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "token buffer allocation failed");
    }
    *n = (int64_t)ids.size();
    if ((int64_t)ids.size() > capacity)
        return tzh_fail(TZH_ERR_TOO_LARGE, "%zu tokens do not fit a capacity of %lld", ids.size(),
                        (long long)capacity);
    if (!ids.empty()) std::memcpy(out, ids.data(), ids.size() * 4);
    return TZH_OK;
}
