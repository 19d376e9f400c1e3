// tokenizers.h — the text front ends of the reference pipeline (host C++): CLIP byte-level BPE and
// the T5 sentencepiece unigram segmentation, with the reference's exact rules
// (src/tokenizers.h:12-31, src/tokenizers.cpp), vocabularies read from the tokenizer GGUFs'
// array metadata (clip.vocab / clip.merges, t5.pieces / t5.scores).
#pragma once
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace tsn {

class ClipBpe {
public:
    int load(const char *gguf_path);
    // bos, byte-level BPE of each lowercased whitespace-separated word (last symbol + "</w>"),
    // eos; cut to ctx (last id eos) or padded with eos to ctx
    std::vector<int32_t> encode(const std::string &text, int ctx) const;
    // vocabulary and merge list given directly (test and embedding use)
    void set(const std::vector<std::string> &vocab, const std::vector<std::string> &merges, int32_t bos,
             int32_t eos);

    int32_t bos = 49406, eos = 49407;

private:
    std::unordered_map<std::string, int32_t> vocab_, rank_;
    std::string byte_sym_[256];   // byte -> its printable unicode symbol (UTF-8)
    void build_byte_table();
};

class T5Unigram {
public:
    int load(const char *gguf_path);
    // trimmed text, spaces as U+2581 with one leading U+2581, best-scoring segmentation into
    // pieces (unknown characters at min(score, 0) - 10 each), eos; cut to ctx (last id eos),
    // padded with pad_id to ctx when pad
    std::vector<int32_t> encode(const std::string &text, int ctx, bool pad) const;
    void set(const std::vector<std::string> &pieces, const std::vector<float> &scores, int32_t unk, int32_t eos,
             int32_t pad);

    int32_t unk_id = 2, eos_id = 1, pad_id = 0;

private:
    std::vector<float> scores_;
    std::unordered_map<std::string, int32_t> id_;
    double unk_score_ = -10.0;
};

} // namespace tsn
