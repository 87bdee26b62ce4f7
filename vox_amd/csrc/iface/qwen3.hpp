// qwen3.hpp — the part of Vox's Qwen3-TTS weight holder that the device backend reads (the codec decoder's layers),
// restated so that gpu_hip.cpp builds on its own. In Vox itself gpu_hip.cpp is compiled against Vox's own
// src/qwen3.hpp; the declarations here keep its names, member order and meaning (reference: src/qwen3.hpp:14-104).
// Only data members are restated (the class has no virtual functions, so its methods do not change its layout).
#pragma once
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "kernels.hpp"

namespace vox {

class TmodFile;

struct TalkerCfg {
    int hidden = 0, inter = 0, layers = 0, heads = 0, kv_heads = 0, head_dim = 0, vocab = 0;
    int text_hidden = 0, text_vocab = 0, groups = 0;
    float eps = 1e-6f;
    double theta = 1e6;
    int eos = 0, think = 0, nothink = 0, think_bos = 0, think_eos = 0, pad = 0, bos = 0;
    std::map<std::string, int> lang;
    std::map<std::string, int> spk_id;
    std::map<std::string, std::string> spk_dialect;
};
struct PredCfg {
    int hidden = 0, inter = 0, layers = 0, heads = 0, kv_heads = 0, head_dim = 0, vocab = 0;
    float eps = 1e-6f;
    double theta = 1e6;
};
struct CodecCfg {
    int codebook_size = 0, hidden = 0, latent = 0, heads = 0, kv_heads = 0, head_dim = 0, window = 0, inter = 0;
    int layers = 0, quantizers = 0, decoder_dim = 0, codebook_dim = 0;
    float layer_scale = 0.01f, eps = 1e-5f;
    double theta = 10000.0;
    std::vector<int> up_rates, up_ratios;
};
struct SpecialIds { int im_start = 0, im_end = 0, tts_pad = 0, tts_bos = 0, tts_eos = 0; };

struct CConv { Mat w; int K = 1, cin = 0, cout = 0, dil = 1; };            // w: [cout][K cin] (+ bias)
struct CDw { const float *w = nullptr, *b = nullptr; int K = 7, C = 0; };  // depthwise: w [C][K]
struct CTrans { Mat w; int K = 0, stride = 1, cin = 0, cout = 0; };        // w: [K cout][cin]
struct Snake { std::vector<float> a, inv_b; };                             // exp(alpha), 1 / (exp(beta) + 1e-9)

class Qwen3Weights {
public:
    std::shared_ptr<TmodFile> file;
    TalkerCfg tc;
    PredCfg pc;
    CodecCfg cc;
    SpecialIds ids;
    TransformerW talker;
    Mat codec_emb, text_emb, codec_head, tp1, tp2;
    TransformerW pred;
    std::vector<Mat> pred_emb, pred_head;
    Mat small_proj;
    bool has_small = false;
    int codec_gpu = -1;
    std::vector<Mat> q_first, q_rest;
    Mat q_first_out, q_rest_out;
    CConv pre_conv;
    Mat pt_in, pt_out;
    TransformerW pt;
    struct UpStage { CTrans tr; const float *tr_b = nullptr; CDw dw; const float *ln_w = nullptr, *ln_b = nullptr, *gamma = nullptr; Mat pw1, pw2; };
    std::vector<UpStage> up;
    CConv conv0;
    struct DecBlock { Snake act; CTrans tr; const float *tr_b = nullptr; Snake a1[3], a2[3]; CConv c1[3], c2[3]; };
    std::vector<DecBlock> blocks;
    Snake final_act;
    CConv final_conv;
};

}  // namespace vox
