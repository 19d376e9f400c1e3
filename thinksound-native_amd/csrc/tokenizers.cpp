// tokenizers.cpp — CLIP BPE and T5 unigram tokenizers (host C++).
#include "tokenizers.h"

#include <limits.h>

#include <algorithm>

#include "gguf.h"
#include "tsn_common.h"

namespace tsn {

namespace {

// UTF-8 encoding of a code point below 0x10000
std::string utf8_of(int cp) {
    std::string s;
    if (cp < 0x80) {
        s += (char)cp;
    } else if (cp < 0x800) {
        s += (char)(0xC0 | (cp >> 6));
        s += (char)(0x80 | (cp & 0x3F));
    } else {
        s += (char)(0xE0 | (cp >> 12));
        s += (char)(0x80 | ((cp >> 6) & 0x3F));
        s += (char)(0x80 | (cp & 0x3F));
    }
    return s;
}

// split into UTF-8 characters by the lead byte (1, 2, 3 or 4 bytes; a cut last character is kept)
std::vector<std::string> utf8_split(const std::string &s) {
    std::vector<std::string> out;
    size_t i = 0;
    while (i < s.size()) {
        const unsigned char c = (unsigned char)s[i];
        const size_t n = c < 0x80 ? 1 : (c >> 5) == 0x6 ? 2 : (c >> 4) == 0xE ? 3 : 4;
        out.push_back(s.substr(i, n));
        i += n;
    }
    return out;
}

bool is_space(unsigned char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\v' || c == '\f' || c == '\r'; }

} // namespace

/* ---------------- CLIP ---------------- */

// GPT-2's printable byte alphabet: '!'..'~', 0xA1..0xAC and 0xAE..0xFF map to themselves; the
// other 68 bytes, in increasing order, to U+0100, U+0101, ...
void ClipBpe::build_byte_table() {
    int next = 256;
    for (int b = 0; b < 256; ++b) {
        const bool printable = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
        byte_sym_[b] = utf8_of(printable ? b : next++);
    }
}

void ClipBpe::set(const std::vector<std::string> &vocab, const std::vector<std::string> &merges, int32_t b,
                  int32_t e) {
    vocab_.clear();
    rank_.clear();
    for (size_t i = 0; i < vocab.size(); ++i) vocab_[vocab[i]] = (int32_t)i;   // a repeated entry: last index wins
    for (size_t i = 0; i < merges.size(); ++i) rank_[merges[i]] = (int32_t)i;
    bos = b;
    eos = e;
    build_byte_table();
}

int ClipBpe::load(const char *path) {
    GgufReader g;
    TSN_TRY(g.open(path));
    const auto &v = g.get_arr_str("clip.vocab");
    TSN_REQUIRE(!v.empty(), std::string("clip tokenizer: no clip.vocab in ") + path);
    set(v, g.get_arr_str("clip.merges"), (int32_t)g.get_i64("clip.bos_id", 49406),
        (int32_t)g.get_i64("clip.eos_id", 49407));
    return TSN_OK;
}

std::vector<int32_t> ClipBpe::encode(const std::string &text, int ctx) const {
    std::vector<int32_t> ids{bos};
    std::string word;
    auto flush = [&]() {
        if (word.empty()) return;
        std::vector<std::string> sym;
        for (unsigned char b : word) sym.push_back(byte_sym_[b]);
        sym.back() += "</w>";
        // merge the lowest-ranked adjacent pair (the leftmost of equal ranks) until none is listed
        while (sym.size() > 1) {
            int best = INT_MAX;
            size_t at = 0;
            for (size_t i = 0; i + 1 < sym.size(); ++i) {
                const auto it = rank_.find(sym[i] + " " + sym[i + 1]);
                if (it != rank_.end() && it->second < best) {
                    best = it->second;
                    at = i;
                }
            }
            if (best == INT_MAX) break;
            sym[at] += sym[at + 1];
            sym.erase(sym.begin() + (long)at + 1);
        }
        for (const auto &t : sym) {
            const auto it = vocab_.find(t);
            if (it != vocab_.end()) ids.push_back(it->second);   // symbols outside the vocabulary are dropped
        }
        word.clear();
    };
    for (char ch : text) {
        const unsigned char c = (unsigned char)ch;
        if (is_space(c)) flush();
        else word += (char)((c >= 'A' && c <= 'Z') ? c + ('a' - 'A') : c);
    }
    flush();
    ids.push_back(eos);
    if ((int)ids.size() > ctx) {
        ids.resize((size_t)ctx);
        ids.back() = eos;
    }
    while ((int)ids.size() < ctx) ids.push_back(eos);
    return ids;
}

/* ---------------- T5 ---------------- */

void T5Unigram::set(const std::vector<std::string> &pieces, const std::vector<float> &scores, int32_t unk,
                    int32_t e, int32_t p) {
    id_.clear();
    for (size_t i = 0; i < pieces.size(); ++i) id_[pieces[i]] = (int32_t)i;   // last index wins
    scores_.assign(pieces.size(), 0.0f);
    for (size_t i = 0; i < pieces.size() && i < scores.size(); ++i) scores_[i] = scores[i];
    double lo = 0.0;
    for (float s : scores_) lo = std::min(lo, (double)s);
    unk_score_ = lo - 10.0;
    unk_id = unk;
    eos_id = e;
    pad_id = p;
}

int T5Unigram::load(const char *path) {
    GgufReader g;
    TSN_TRY(g.open(path));
    const auto &pieces = g.get_arr_str("t5.pieces");
    TSN_REQUIRE(!pieces.empty(), std::string("t5 tokenizer: no t5.pieces in ") + path);
    const auto sc = g.get_arr_num("t5.scores");
    std::vector<float> scores(sc.begin(), sc.end());
    set(pieces, scores, (int32_t)g.get_i64("t5.unk_id", 2), (int32_t)g.get_i64("t5.eos_id", 1),
        (int32_t)g.get_i64("t5.pad_id", 0));
    return TSN_OK;
}

std::vector<int32_t> T5Unigram::encode(const std::string &text, int ctx, bool pad) const {
    static const std::string SP = "\xE2\x96\x81";   // U+2581, the word-boundary mark
    const size_t a = text.find_first_not_of(" \t\n"), b = text.find_last_not_of(" \t\n");
    const std::string body = a == std::string::npos ? std::string() : text.substr(a, b - a + 1);
    std::string t = SP;
    for (char ch : body) {
        if (ch == ' ') t += SP;
        else t += ch;
    }
    const std::vector<std::string> ch = utf8_split(t);
    const int L = (int)ch.size();
    // best[i]: best score of a segmentation of the first i characters; from[i], tok[i]: its last step
    std::vector<double> best((size_t)L + 1, -1e18);
    std::vector<int> from((size_t)L + 1, -1), tok((size_t)L + 1, -1);
    best[0] = 0.0;
    for (int i = 0; i < L; ++i) {
        if (best[i] <= -1e17) continue;
        std::string piece;
        for (int j = i; j < L; ++j) {
            piece += ch[j];
            const auto it = id_.find(piece);
            if (it != id_.end()) {
                const double s = best[i] + scores_[it->second];
                if (s > best[j + 1]) {
                    best[j + 1] = s;
                    from[j + 1] = i;
                    tok[j + 1] = it->second;
                }
            }
            if (piece.size() > 64) break;
        }
        const double s = best[i] + unk_score_;
        if (s > best[i + 1]) {
            best[i + 1] = s;
            from[i + 1] = i;
            tok[i + 1] = unk_id;
        }
    }
    std::vector<int32_t> ids;
    for (int i = L; i > 0;) {
        ids.push_back(tok[i]);
        if (from[i] < 0) break;
        i = from[i];
    }
    std::reverse(ids.begin(), ids.end());
    ids.push_back(eos_id);
    if ((int)ids.size() > ctx) {
        ids.resize((size_t)ctx);
        ids.back() = eos_id;
    }
    if (pad)
        while ((int)ids.size() < ctx) ids.push_back(pad_id);
    return ids;
}

} // namespace tsn
