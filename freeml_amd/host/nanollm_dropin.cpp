// NanoLLM through FreeML's own Model / Datablob / MatrixManager / Layer API on a selectable
// backend: MatrixCPU<float> (the reference) or MatrixHIP<float> (this backend).
//
// The graph is built with the same sequence of reference API calls as BuildOrLoadModel
// (Examples/NanoLLM/NanoLLM.cpp:255-376) and run with Model::Run (Model.h:764-788), one
// padded block_size window per greedy step (the token history padded with id 0, logits row
// len-1, first-max argmax, NanoLLM.cpp:189-205).  Weights come from a file so both backends see identical
// parameters.  Compiled against the reference headers (freeml_amd/host/Makefile).
//
// Usage: nanollm_dropin <cpu|hip|hiploop|cpuhip> <in.bin> <out.bin> [--load DIR] [--save DIR]
//                       [--train K [--grads]] [--bias] [--dropout P]
//   hiploop: the graph is built on MatrixHIP as for `hip`, then NanoLLMTokenLoop decodes
//   from the blobs' device matrices with the KV-cache loop instead of Model::Run.
//   --load DIR: the model comes from the FreeML checkpoint DIR/NanoLLM_dropin written by
//   Model::Save (the BuildOrLoadModel load branch, NanoLLM.cpp:264-268 + 357-360, then the
//   position input of NanoLLM.cpp:383-402); in.bin then supplies only the prompt and n_gen
//   (its parameter arrays are read and ignored).
//   --save DIR: after generation, Model::Save writes the model (every blob matrix, with an
//   AdamW optimiser attached as NanoLLM.cpp:353-355 does) to DIR/NanoLLM_dropin, through
//   the backend's GetRawData.
//   --bias / --dropout P: the graph built with biases in the blocks' Dense layers (useBias) and
//   dropout probability P in the embedding, attention-residual and MLP dropout layers (NanoLLM
//   uses neither; the attention-weight dropout stays off, see Build).
//   cpuhip (with --train): the K iterations on MatrixCPU, then on MatrixHIP, in this one
//   process (the dropout masks of both then come from the same RandomUtils uniform buffer);
//   out.bin holds MatrixHIP's results, out.bin.cpu MatrixCPU's.
//   --train K: instead of generating, K training iterations of NanoLLM's TrainLoop
//   (NanoLLM.cpp:416-445): the prompt is the corpus (at least T+1 ids); iteration k copies the
//   window at start_k = (7919 k) mod (P - T) and its one-token-shifted target out of the corpus
//   matrix with CopyRange, then Model::Run(window, target, storeLoss = true) runs forward, the
//   CategoricalCrossEntropyWithLogits gradient, the backward and AdamW (lr 1e-4, betas
//   0.9/0.999, eps 1e-8, weight decay 0.01: NanoLLM.cpp:56, :353-355).  With --grads no
//   optimiser is attached, so the gradients stay in the blobs for --save.  out.bin is then
//   float64 losses (K), float64 wall seconds per iteration (K; the device is synchronised at
//   the end of each) and the uint64 {d2h, h2d} copy counts of iterations 1..K-1.
//   in.bin:  int32[9] {V, T, C, H, L, tied, P, n_gen, unused}, then float32 tok_emb (V*C),
//            pos_emb (T*C), per layer w_qkv (C*3C), w_proj (C*C), w_fc (C*4C), w_proj2 (4C*C),
//            ln0_gamma (C), ln1_gamma (C); lnf_gamma (C); lm_head (V*C) when not tied;
//            int32 prompt (P).
//   out.bin: int32 tokens (n_gen), float32 logits (n_gen*V), uint64 {d2h, h2d} copies made
//            by MatrixHIP during steps 1..n_gen-1 (step 0 uploads the host-written weights);
//            a forward with every op on the device makes exactly one of each per step: the
//            input window up, the logits down.  0 for cpu.
#include <ModelLibrary/Model.h>
#include <LayerLibrary/Layers.h>
#include <LossLibrary/Losses.h>
#include <OptimiserLibrary/Optimisers.h>
#include <MatrixLibrary/CPU/MatrixCPU.h>
#include <MatrixLibrary/GPU/HIP/MatrixHIP.h>
#include <MatrixLibrary/GPU/HIP/MatrixHIP_Functions.h>
#include <MatrixLibrary/GPU/HIP/NanoLLMTokenLoop.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <memory>
#include <string>
#include <type_traits>
#include <vector>

namespace {

struct Params {
    int32_t V, T, C, H, L, tied, P, n_gen, unused;
    std::vector<float> tok, pos, lnf, lm;
    std::vector<std::vector<float>> qkv, proj, fc, proj2, ln0, ln1;
    std::vector<int32_t> prompt;
    bool bias = false;     // --bias: the blocks' Dense layers with biases (useBias)
    float dropout = 0.f;   // --dropout P: the embedding's and the blocks' dropout probability
};

template <class V>
bool ReadVec(std::ifstream& f, V& v, size_t n) {
    v.resize(n);
    f.read(reinterpret_cast<char*>(v.data()), n * sizeof(typename V::value_type));
    return static_cast<bool>(f);
}

bool ReadParams(const char* path, Params& p) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    f.read(reinterpret_cast<char*>(&p.V), 9 * sizeof(int32_t));
    const size_t C = p.C;
    bool ok = ReadVec(f, p.tok, (size_t)p.V * C) && ReadVec(f, p.pos, (size_t)p.T * C);
    p.qkv.resize(p.L); p.proj.resize(p.L); p.fc.resize(p.L); p.proj2.resize(p.L);
    p.ln0.resize(p.L); p.ln1.resize(p.L);
    for (int l = 0; ok && l < p.L; ++l)
        ok = ReadVec(f, p.qkv[l], C * 3 * C) && ReadVec(f, p.proj[l], C * C) && ReadVec(f, p.fc[l], C * 4 * C) &&
             ReadVec(f, p.proj2[l], 4 * C * C) && ReadVec(f, p.ln0[l], C) && ReadVec(f, p.ln1[l], C);
    ok = ok && ReadVec(f, p.lnf, C);
    if (ok && !p.tied) ok = ReadVec(f, p.lm, (size_t)p.V * C);
    return ok && ReadVec(f, p.prompt, (size_t)p.P);
}

template <class Mat>
void Write(Mat* m, const std::vector<float>& src) {
    assert(m && m->GetElementCount() == src.size());
    std::memcpy(m->DataWrite(), src.data(), src.size() * sizeof(float));
}

template <class Mat>
struct Graph {
    using MatrixRef = typename MatrixManager<float, Mat>::MatrixRef;
    std::unique_ptr<Model<float, Mat>> model;
    MatrixRef posInput, input, untied;
};

constexpr const char* kModelName = "NanoLLM_dropin";

// Position ids 0..T-1 into embedding_pos (NanoLLM.cpp:383-402).
template <class Mat>
void SetPositions(Graph<Mat>& g, uint32_t Tb) {
    auto& inst = MatrixManager<float, Mat>::Instance();
    g.posInput = inst.AllocateMatrix({1u, Tb, 1u}, "Pos_Input");
    for (uint32_t t = 0; t < Tb; ++t) g.posInput->SetValue(0u, t, 0u, static_cast<float>(t));
    g.model->GetLayer("embedding_pos")
        ->SetInput(g.model->GetLayerBlob("embedding_pos"), g.posInput.get(), 0u);
}

// The NanoLLM graph of NanoLLM.cpp:267-358 on backend Mat, with the given parameters.  With
// `optimiser`, the AdamW optimiser of NanoLLM.cpp:353-355 is attached, so Model::Save writes
// the same kinds of files a training run's checkpoint holds.
template <class Mat>
Graph<Mat> Build(const Params& p, bool optimiser) {
    using T = float;
    auto& inst = MatrixManager<T, Mat>::Instance();
    Graph<Mat> g;
    g.model = std::make_unique<Model<T, Mat>>();
    auto* model = g.model.get();
    const uint32_t V = p.V, Tb = p.T, C = p.C, H = p.H, B = 1;

    auto* tok = new Embedding<T, Mat>();
    tok->SetName("embedding_token");
    auto* tokBlob = InitEmbeddingBlob<T, Mat>(V, C, Tb, B, true);
    model->AddLayer(tok, tokBlob);
    auto* pos = new Embedding<T, Mat>();
    pos->SetName("embedding_pos");
    model->AddLayer(pos, InitEmbeddingBlob<T, Mat>(Tb, C, Tb, B, true));
    auto* add = new AddLayer<T, Mat>();
    add->SetName("token_pos_add");
    model->AddLayer(add, InitAddBlob<T, Mat>(true));
    model->AddDependency(add, 0, tok, 0);
    model->AddDependency(add, 1, pos, 0);
    auto* drop = new DropoutLayer<T, Mat>();
    drop->SetName("embedding_dropout");
    model->AddLayer(drop, InitDropoutBlob<T, Mat>(p.dropout, true));
    model->AddDependency(drop, 0, add, 0);
    Layer<T, Mat>* prev = drop;
    for (int l = 0; l < p.L; ++l) {
        auto* blk = new TransformerBlockLayer<T, Mat>();
        blk->SetName("block_" + std::to_string(l));
        const float residProjScale = 1.0f / std::sqrt(2.0f * static_cast<float>(p.L));
        model->AddLayer(blk, InitTransformerBlockBlob<T, Mat>(C, H, p.dropout, Tb, B, true, p.bias, residProjScale));
        model->AddDependency(blk, 0, prev, 0);
        prev = blk;
    }
    auto* lnf = new LayerNorm<T, Mat>();
    lnf->SetName("ln_f");
    model->AddLayer(lnf, InitLayerNormBlob<T, Mat>(true, true, false));
    model->AddDependency(lnf, 0, prev, 0);
    auto* flat = new FlattenCopyLayer<T, Mat>();
    flat->SetName("ln_f_flatten");
    model->AddLayer(flat, InitFlattenCopyBlob<T, Mat>(true));
    model->AddDependency(flat, 0, lnf, 0);
    auto* head = new Dense<T, Identity<T>, Mat, true>();
    head->SetName("lm_head");
    auto* headBlob = InitDenseBlob<T, Mat>(V, C, Tb * B, true, true, false, true);
    // Tie lm_head to the token embedding (NanoLLM.cpp:333-345).
    Mat* headW = headBlob->template GetMatrix<Mat>("Dense_Weights");
    headBlob->Set("Dense_Weights", inst.GetHandle(tokBlob->template GetMatrix<Mat>("Embedding_Weights")));
    inst.RemoveMatrix(headW);
    model->AddLayer(head, headBlob);
    model->AddDependency(head, 0, flat, 0);
    model->SetFinalOutputLayer(head);
    if (optimiser) model->SetOptimiser(new AdamWOptimiser<T, Mat>(1e-4f, 0.9f, 0.999f, 1e-8f, 0.01f));
    model->SetLoss(new CategoricalCrossEntropyWithLogits<T, Mat>());
    model->SetExpectedInputDims({1u, Tb, B});
    model->SetName(kModelName);
    model->Init();
    SetPositions(g, Tb);

    // Parameters (the random init and residProjScale above are overwritten).
    Write(model->GetLayerBlob("embedding_token")->GetMatrix("Embedding_Weights"), p.tok);
    Write(model->GetLayerBlob("embedding_pos")->GetMatrix("Embedding_Weights"), p.pos);
    for (int l = 0; l < p.L; ++l) {
        auto* blk = model->GetLayerBlob("block_" + std::to_string(l));
        auto* att = blk->GetBlob("AttentionLayerData");
        Write(blk->GetBlob("LayerNorm0Data")->GetMatrix("GammaScale"), p.ln0[l]);
        Write(att->GetBlob("CSA_AttentionLayer")->GetMatrix("Dense_Weights"), p.qkv[l]);
        Write(att->GetBlob("CSA_ProjLayer")->GetMatrix("Dense_Weights"), p.proj[l]);
        Write(blk->GetBlob("LayerNorm1Data")->GetMatrix("GammaScale"), p.ln1[l]);
        Write(blk->GetBlob("DenseFCData")->GetMatrix("Dense_Weights"), p.fc[l]);
        Write(blk->GetBlob("DenseProjData")->GetMatrix("Dense_Weights"), p.proj2[l]);
        // Dropout on the attention weights stays off: its backward cannot run on the
        // reference's MatrixCPU (CausalSelfAttentionLayer.h:593, :638 passes a local view to
        // SetErrorInput, which asserts at Datablob.h:245 because no MatrixManager handle owns
        // it).  Its layers become identities (probability 0, scale 1); the embedding,
        // residual and MLP dropouts keep --dropout.
        for (int hh = 0; p.dropout > 0.f && hh < p.H; ++hh) {
            auto* d = att->GetBlob("CSA_AttentionDropout_" + std::to_string(hh));
            if (!d) continue;
            d->Set("Probability", 0.0f);
            Write(d->GetMatrix("ScalarScale"), std::vector<float>{1.0f});
        }
    }
    Write(model->GetLayerBlob("ln_f")->GetMatrix("GammaScale"), p.lnf);
    if (!p.tied) {
        g.untied = inst.AllocateMatrix({C, V}, "Dense_Weights");
        Write(g.untied.get(), p.lm);
        model->GetLayerBlob("lm_head")->Set("Dense_Weights", g.untied);
    }
    g.input = inst.AllocateMatrix({1u, Tb, 1u}, "Input_Window");
    return g;
}

// Model::Load / Model::Save run with the working directory at `dir`: both resolve the
// checkpoint folder as current_path()/<model name> (Model.h:91-96, :161-170).
class InDir {
public:
    explicit InDir(const std::string& dir) : old_(std::filesystem::current_path()) {
        std::filesystem::create_directories(dir);
        std::filesystem::current_path(dir);
    }
    ~InDir() { std::filesystem::current_path(old_); }
private:
    std::filesystem::path old_;
};

// The load branch of BuildOrLoadModel (NanoLLM.cpp:264-268, :357-360): every layer, blob and
// matrix comes from the checkpoint's files through SaveLoader, which writes each matrix with
// DataWrite (SaveLoader.h:1350-1397) and resolves the tied lm_head by GUID.
template <class Mat>
bool Load(const Params& p, const std::string& dir, Graph<Mat>& g) {
    g.model = std::make_unique<Model<float, Mat>>();
    {
        InDir in(dir);
        if (!g.model->Load(kModelName)) return false;
    }
    g.model->Init();
    if (!g.model->GetLayer("embedding_pos") || !g.model->GetLayerBlob("lm_head")) return false;
    SetPositions(g, static_cast<uint32_t>(p.T));
    g.input = MatrixManager<float, Mat>::Instance().AllocateMatrix({1u, static_cast<uint32_t>(p.T), 1u},
                                                                   "Input_Window");
    return true;
}

template <class Mat>
int Run(Graph<Mat>& g, const Params& p, std::vector<int32_t>& tokens, std::vector<float>& logits,
        uint64_t copies[2]) {
    const uint32_t T = p.T, V = p.V;
    std::vector<int32_t> hist(p.prompt.begin(), p.prompt.end());
    tokens.assign(p.n_gen, 0);
    logits.assign((size_t)p.n_gen * V, 0.f);
    copies[0] = copies[1] = 0;
    for (int s = 0; s < p.n_gen; ++s) {
        // Window: history padded with id 0 (every valid row is independent of the padding).
        float* in = g.input->DataWrite();
        for (uint32_t t = 0; t < T; ++t) in[t] = t < hist.size() ? static_cast<float>(hist[t]) : 0.f;
        const freeml_hip::TransferStats before = freeml_hip::Stats();
        g.model->Run(g.input.get(), nullptr);
        Mat* out = g.model->GetOutput();
        if (!out || out->GetDimsX() != V || out->GetDimsY() != T) return 2;
        const float* row = out->DataRead() + (size_t)(hist.size() - 1) * V;
        const freeml_hip::TransferStats after = freeml_hip::Stats();
        if (s > 0) {
            copies[0] += after.toHost - before.toHost;
            copies[1] += after.toDevice - before.toDevice;
        }
        std::memcpy(&logits[(size_t)s * V], row, V * sizeof(float));
        uint32_t best = 0;
        float bv = row[0];
        for (uint32_t v = 1; v < V; ++v)
            if (row[v] > bv) { bv = row[v]; best = v; }
        tokens[s] = static_cast<int32_t>(best);
        if (hist.size() < T) hist.push_back(static_cast<int32_t>(best));
    }
    return 0;
}

int RunLoop(Graph<MatrixHIP<float>>& g, const Params& p, std::vector<int32_t>& tokens,
            std::vector<float>& logits) {
    freeml_hip::NanoLLMTokenLoop loop;
    if (!loop.Create(g.model.get(), 1)) return 5;
    if (!loop.Generate(p.prompt, 1, p.n_gen, tokens, &logits)) return 6;
    return 0;
}

template <class Mat>
void Sync() {
    if constexpr (std::is_same_v<Mat, MatrixHIP<float>>) freeml_hip::Check(fmlh_synchronize(), "fmlh_synchronize");
}

template <class Mat>
int Train(Graph<Mat>& g, const Params& p, int steps, std::vector<double>& losses, std::vector<double>& secs,
          uint64_t copies[2]) {
    const uint32_t T = p.T, P = static_cast<uint32_t>(p.prompt.size());
    if (P < T + 1) return 11;
    auto& inst = MatrixManager<float, Mat>::Instance();
    auto corpus = inst.AllocateMatrix({1u, P, 1u}, "Corpus_Tokens");
    float* c = corpus->DataWrite();
    for (uint32_t i = 0; i < P; ++i) c[i] = static_cast<float>(p.prompt[i]);
    auto target = inst.AllocateMatrix({1u, T, 1u}, "Target_Buffer");
    const uint32_t span = P - T;
    copies[0] = copies[1] = 0;
    for (int s = 0; s < steps; ++s) {
        const uint32_t start = static_cast<uint32_t>((7919ull * static_cast<uint64_t>(s)) % span);
        const freeml_hip::TransferStats before = freeml_hip::Stats();
        const auto t0 = std::chrono::steady_clock::now();
        CopyRange(g.input.get(), corpus.get(), 0u, start, T);
        CopyRange(target.get(), corpus.get(), 0u, start + 1u, T);
        g.model->Run(g.input.get(), target.get(), true);
        losses.push_back(static_cast<double>(g.model->GetLastLoss()));
        Sync<Mat>();
        secs.push_back(std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
        const freeml_hip::TransferStats after = freeml_hip::Stats();
        if (s > 0) {
            copies[0] += after.toHost - before.toHost;
            copies[1] += after.toDevice - before.toDevice;
        }
    }
    return 0;
}

template <class Mat>
int Execute(const std::string& backend, const Params& p, const std::string& load_dir,
            const std::string& save_dir, int train_steps, bool grads_only, std::vector<int32_t>& tokens,
            std::vector<float>& logits, std::vector<double>& losses, std::vector<double>& secs,
            uint64_t copies[2]) {
    Graph<Mat> g;
    if (!load_dir.empty()) {
        if (!Load(p, load_dir, g)) {
            std::fprintf(stderr, "cannot load %s/%s\n", load_dir.c_str(), kModelName);
            return 7;
        }
        // SaveLoader rebuilds every Dense as Dense<T, Act, Mat> with TransposedWeights = false
        // (SaveLoader.h:1015-1043; Dense::GetMetaData stores only the activation name,
        // Dense.h:173-177), so the reloaded lm_head no longer reads its {C, V} weights
        // transposed (NanoLLM.cpp:328) and Model::Run stops at the product's dimension check
        // (MatrixBase_Mul.h:497 on MatrixCPU).  The token loop reads the blob matrices by name
        // and is unaffected.
        const bool run_graph = backend != "hiploop" || train_steps > 0;
        if (run_graph && !dynamic_cast<Dense<float, Identity<float>, Mat, true>*>(g.model->GetLayer("lm_head"))) {
            std::fprintf(stderr,
                         "%s: the reloaded lm_head is Dense<..., TransposedWeights=false>; Model::Run "
                         "cannot run this checkpoint (decode it with hiploop)\n",
                         load_dir.c_str());
            return 10;
        }
    } else {
        g = Build<Mat>(p, train_steps > 0 ? !grads_only : !save_dir.empty());
    }
    int rc;
    if (train_steps > 0) {
        rc = Train(g, p, train_steps, losses, secs, copies);
    } else if constexpr (std::is_same_v<Mat, MatrixHIP<float>>) {
        rc = backend == "hiploop" ? RunLoop(g, p, tokens, logits) : Run(g, p, tokens, logits, copies);
    } else {
        rc = Run(g, p, tokens, logits, copies);
    }
    if (rc || save_dir.empty()) return rc;
    InDir in(save_dir);
    return g.model->Save() ? 0 : 8;
}

}  // namespace

int main(int argc, char** argv) {
    std::string load_dir, save_dir;
    int train_steps = 0;
    bool grads_only = false, use_bias = false;
    float dropout = 0.f;
    int npos = 0;
    const char* pos[3] = {nullptr, nullptr, nullptr};
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if ((a == "--load" || a == "--save") && i + 1 < argc) {
            (a == "--load" ? load_dir : save_dir) = argv[++i];
        } else if (a == "--train" && i + 1 < argc) {
            train_steps = std::atoi(argv[++i]);
        } else if (a == "--grads") {
            grads_only = true;
        } else if (a == "--bias") {
            use_bias = true;
        } else if (a == "--dropout" && i + 1 < argc) {
            dropout = static_cast<float>(std::atof(argv[++i]));
        } else if (npos < 3) {
            pos[npos++] = argv[i];
        } else {
            npos = 4;
        }
    }
    const std::string backend = npos == 3 ? pos[0] : "";
    if ((backend != "cpu" && backend != "hip" && backend != "hiploop" && backend != "cpuhip") ||
        train_steps < 0 || (grads_only && train_steps == 0) || (backend == "cpuhip" && train_steps == 0) ||
        dropout < 0.f || dropout >= 1.f) {
        std::fprintf(stderr,
                     "usage: %s <cpu|hip|hiploop|cpuhip> <in.bin> <out.bin> [--load DIR] [--save DIR] "
                     "[--train K [--grads]] [--bias] [--dropout P]\n",
                     argv[0]);
        return 1;
    }
    Tools::Logger::EnableConsole(false);
    Params p;
    if (!ReadParams(pos[1], p)) {
        std::fprintf(stderr, "cannot read %s\n", pos[1]);
        return 1;
    }
    p.bias = use_bias;
    p.dropout = dropout;
    std::vector<int32_t> tokens;
    std::vector<float> logits;
    std::vector<double> losses, secs;
    uint64_t copies[2] = {0, 0};
    int rc;
    if (backend == "cpuhip") {
        // MatrixCPU first, into out.bin.cpu (losses, seconds, zero copies), then MatrixHIP below.
        std::vector<double> cl, cs;
        uint64_t cc[2] = {0, 0};
        rc = Execute<MatrixCPU<float>>("cpu", p, load_dir, save_dir, train_steps, grads_only, tokens, logits,
                                       cl, cs, cc);
        if (rc) return rc;
        std::ofstream fc(std::string(pos[2]) + ".cpu", std::ios::binary);
        fc.write(reinterpret_cast<const char*>(cl.data()), cl.size() * sizeof(double));
        fc.write(reinterpret_cast<const char*>(cs.data()), cs.size() * sizeof(double));
        fc.write(reinterpret_cast<const char*>(cc), sizeof(cc));
        if (!fc) return 4;
    }
    if (backend == "hip" || backend == "hiploop" || backend == "cpuhip") {
        if (fmlh_init(0) != FMLH_OK) {
            std::fprintf(stderr, "fmlh_init: %s\n", fmlh_last_error());
            return 3;
        }
        rc = Execute<MatrixHIP<float>>(backend == "cpuhip" ? "hip" : backend, p, load_dir, save_dir, train_steps,
                                       grads_only, tokens, logits, losses, secs, copies);
    } else {
        rc = Execute<MatrixCPU<float>>(backend, p, load_dir, save_dir, train_steps, grads_only, tokens,
                                       logits, losses, secs, copies);
    }
    if (rc) return rc;
    std::ofstream f(pos[2], std::ios::binary);
    if (backend != "cpu") {
        const freeml_hip::AttentionCounts& a = freeml_hip::AttnCounts();
        std::printf("attention layer: %llu batched / %llu per-head forwards, %llu batched / %llu per-head backwards\n",
                    (unsigned long long)a.batchedForward, (unsigned long long)a.perHeadForward,
                    (unsigned long long)a.batchedBackward, (unsigned long long)a.perHeadBackward);
    }
    if (train_steps > 0) {
        f.write(reinterpret_cast<const char*>(losses.data()), losses.size() * sizeof(double));
        f.write(reinterpret_cast<const char*>(secs.data()), secs.size() * sizeof(double));
        f.write(reinterpret_cast<const char*>(copies), sizeof(copies));
        double rest = 0.0;
        for (size_t i = 1; i < secs.size(); ++i) rest += secs[i];
        std::printf("%s: %d training iterations, loss %.6f -> %.6f, %.3f ms/iteration after the first, "
                    "%llu d2h / %llu h2d copies after the first\n",
                    backend.c_str(), train_steps, losses.front(), losses.back(),
                    secs.size() > 1 ? 1e3 * rest / (double)(secs.size() - 1) : 1e3 * secs[0],
                    (unsigned long long)copies[0], (unsigned long long)copies[1]);
        return f ? 0 : 4;
    }
    f.write(reinterpret_cast<const char*>(tokens.data()), tokens.size() * sizeof(int32_t));
    f.write(reinterpret_cast<const char*>(logits.data()), logits.size() * sizeof(float));
    f.write(reinterpret_cast<const char*>(copies), sizeof(copies));
    std::printf("%s: %d steps, %llu d2h / %llu h2d copies during Model::Run%s%s\n", backend.c_str(), p.n_gen,
                (unsigned long long)copies[0], (unsigned long long)copies[1],
                load_dir.empty() ? "" : ", loaded", save_dir.empty() ? "" : ", saved");
    return f ? 0 : 4;
}
