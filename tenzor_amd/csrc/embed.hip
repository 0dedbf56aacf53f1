// The embed command's two text paths (main.zig:718-1021) on the GPU: host
// tokenization, every chunk or text of the call packed into one batched
// forward, and for documents a pooling kernel that averages each
// document's chunk embeddings and L2-normalises the mean.
#include <algorithm>
#include <atomic>
#include <cstring>
#include <thread>
#include <vector>

#include "common.h"

namespace {

constexpr int HD = 384;                 // hidden size the pooling kernel is written for
constexpr int64_t kMaxSeq = 512;        // main.zig:782
constexpr int64_t kChunk = 510;         // main.zig:783, room for [CLS] and [SEP]
constexpr int64_t kOverlap = 50;        // main.zig:784
constexpr int64_t kStride = kChunk - kOverlap;

int64_t chunk_count(int64_t total) {
    return total <= kChunk ? 1 : 1 + (total - kChunk + kOverlap - 1) / kStride;  // main.zig:803-806
}

// Mean of each document's chunk embeddings, then L2 (main.zig:908-923),
// one wave per document, lane l holding columns l + 64q.  The sums follow
// the reference's order exactly: chunks added in order onto 0, the mean as
// a product with the f32 reciprocal of the count, the squares summed
// column by column from 0 to 383 (every lane forms the same sequential
// sum from shuffled squares), IEEE sqrt and division.
__global__ void __launch_bounds__(256) chunk_mean_l2_kernel(const float *__restrict__ emb, const int *__restrict__ cu,
                                                             int n_docs, float *__restrict__ out) {
    const int d = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (d >= n_docs) return;
    const int c0 = cu[d], c1 = cu[d + 1];
    float v[6] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = c0; c < c1; c++)
#pragma unroll
        for (int q = 0; q < 6; q++) v[q] = v[q] + emb[(int64_t)c * HD + lane + 64 * q];
    const float scale = 1.0f / (float)(c1 - c0);
    float sq[6];
#pragma unroll
    for (int q = 0; q < 6; q++) {
        v[q] = v[q] * scale;
        sq[q] = v[q] * v[q];
    }
    float norm = 0.0f;
#pragma unroll
    for (int q = 0; q < 6; q++)
        for (int l = 0; l < 64; l++) norm = norm + __shfl(sq[q], l, 64);
    norm = sqrtf(norm);
#pragma unroll
    for (int q = 0; q < 6; q++) out[(int64_t)d * HD + lane + 64 * q] = norm > 0.0f ? v[q] / norm : v[q];
}

// Runs fn(i) for i in [0, n) on up to 16 host threads (static blocks).
template <typename F>
bool parallel_for(int n, F fn) {
    const int workers = std::max(1, std::min<int>({n, 16, (int)std::max(1u, std::thread::hardware_concurrency())}));
    std::atomic<bool> failed{false};
    auto run = [&](int w) {
        try {
            for (int i = (int)((int64_t)n * w / workers); i < (int)((int64_t)n * (w + 1) / workers); i++) fn(i);
        } catch (...) {
            failed = true;
        }
    };
    if (workers == 1) {
        run(0);
        return !failed;
    }
    std::vector<std::thread> threads;
    for (int w = 1; w < workers; w++) threads.emplace_back(run, w);
    run(0);
    for (auto &t : threads) t.join();
    return !failed;
}

int check_texts(tzh_model *m, const tzh_tokenizer *tok, const char *const *texts, const int64_t *lens, int32_t n,
                float *outputs) {
    if (!m || !tok) return tzh_fail(TZH_ERR_INVALID_ARGS, "null model or tokenizer");
    if (n < 0 || (n > 0 && (!texts || !lens || !outputs))) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad text arguments");
    for (int32_t i = 0; i < n; i++)
        if (lens[i] < 0 || (lens[i] > 0 && !texts[i]))
            return tzh_fail(TZH_ERR_INVALID_ARGS, "text %d: bad pointer or length", i);
    if (tzh_model_hidden(m) != HD) return tzh_fail(TZH_ERR_INVALID_ARGS, "hidden size %d is not %d", tzh_model_hidden(m), HD);
    return TZH_OK;
}

}  // namespace

extern "C" int tzh_embed_chunk_count(int64_t total_tokens, int64_t *count) {
    tzh_clear_error();
    if (!count || total_tokens < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad chunk-count arguments");
    *count = chunk_count(total_tokens);
    return TZH_OK;
}

extern "C" int tzh_arctic_embed_documents(tzh_model *m, const tzh_tokenizer *tok, const char *const *texts,
                                          const int64_t *lens, int32_t n_docs, float *outputs,
                                          int32_t *chunk_counts) {
    tzh_clear_error();
    TZH_TRY(check_texts(m, tok, texts, lens, n_docs, outputs));
    if (n_docs == 0) return TZH_OK;
    tzh_ctx *ctx = tzh_model_ctx(m);
    TZH_TRY(tzh_ctx_enter(ctx));

    std::vector<std::vector<uint32_t>> pieces((size_t)n_docs);
    if (!parallel_for(n_docs, [&](int d) { tzh_tokenize_raw(tok, (const uint8_t *)texts[d], (size_t)lens[d], pieces[d]); }))
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "tokenization ran out of memory");

    // chunk plan: document d owns chunks cu[d] .. cu[d+1]
    std::vector<int32_t> cu((size_t)n_docs + 1, 0);
    int64_t n_ids = 0;
    for (int32_t d = 0; d < n_docs; d++) {
        const int64_t total = (int64_t)pieces[d].size(), nc = chunk_count(total);
        if (nc == 1 && total > kChunk)
            return tzh_fail(TZH_ERR_TOO_LARGE,
                            "document %d: %lld pieces make one chunk of more than %lld (the reference overruns its "
                            "chunk buffer here)", d, (long long)total, (long long)kChunk);
        if (cu[d] + nc > INT32_MAX / 2) return tzh_fail(TZH_ERR_TOO_LARGE, "too many chunks");
        cu[d + 1] = cu[d] + (int32_t)nc;
        for (int64_t k = 0; k < nc; k++) n_ids += std::min(k * kStride + kChunk, total) - k * kStride + 2;
        if (chunk_counts) chunk_counts[d] = (int32_t)nc;
    }
    const int32_t n_chunks = cu[n_docs];

    // packed ids of every chunk, then the chunk offsets, in one upload
    const size_t ids_bytes = ((size_t)n_ids * 4 + 255) & ~(size_t)255;
    const size_t cu_bytes = ((size_t)(n_docs + 1) * 4 + 255) & ~(size_t)255;
    std::vector<uint32_t> host(ids_bytes / 4 + cu_bytes / 4);
    std::vector<int32_t> lengths((size_t)n_chunks);
    {
        const uint32_t cls = tzh_tokenizer_cls(tok), sep = tzh_tokenizer_sep(tok);
        size_t p = 0;
        for (int32_t d = 0; d < n_docs; d++) {
            const int64_t total = (int64_t)pieces[d].size();
            for (int32_t k = 0; k < cu[d + 1] - cu[d]; k++) {
                const int64_t s = k * kStride, e = std::min(s + kChunk, total);
                host[p++] = cls;
                std::copy(pieces[d].begin() + s, pieces[d].begin() + e, host.begin() + (int64_t)p);
                p += (size_t)(e - s);
                host[p++] = sep;
                lengths[(size_t)(cu[d] + k)] = (int32_t)(e - s + 2);
            }
        }
        std::memcpy(host.data() + ids_bytes / 4, cu.data(), cu.size() * 4);
    }
    void *scratch = nullptr;
    const size_t emb_bytes = (size_t)n_chunks * HD * 4;
    TZH_TRY(tzh_ctx_scratch(ctx, ids_bytes + cu_bytes + emb_bytes, &scratch));
    uint32_t *d_ids = (uint32_t *)scratch;
    const int *d_cu = (const int *)((char *)scratch + ids_bytes);
    float *d_emb = (float *)((char *)scratch + ids_bytes + cu_bytes);
    TZH_HIP(hipMemcpyAsync(d_ids, host.data(), ids_bytes + cu_bytes, hipMemcpyHostToDevice, ctx->stream));
    TZH_HIP(hipStreamSynchronize(ctx->stream));  // the host staging is freed on return

    TZH_TRY(tzh_arctic_forward_batch(m, d_emb, d_ids, lengths.data(), n_chunks, 0));
    hipLaunchKernelGGL(chunk_mean_l2_kernel, dim3((unsigned)((n_docs + 3) / 4)), dim3(256), 0, ctx->stream, d_emb,
                       d_cu, n_docs, outputs);
    TZH_LAUNCHED("chunk_mean_l2_kernel");
    return TZH_OK;
}

extern "C" int tzh_arctic_embed_texts(tzh_model *m, const tzh_tokenizer *tok, const char *const *texts,
                                      const int64_t *lens, int32_t n_texts, float *outputs, int32_t *n_tokens) {
    tzh_clear_error();
    TZH_TRY(check_texts(m, tok, texts, lens, n_texts, outputs));
    if (n_texts == 0) return TZH_OK;
    tzh_ctx *ctx = tzh_model_ctx(m);
    TZH_TRY(tzh_ctx_enter(ctx));

    // encode into fixed 512-id rows (main.zig:945-954), then pack
    std::vector<uint32_t> rows((size_t)n_texts * kMaxSeq);
    std::vector<int32_t> lengths((size_t)n_texts);
    if (!parallel_for(n_texts, [&](int i) {
            lengths[i] = (int32_t)tzh_tokenize(tok, (const uint8_t *)texts[i], (size_t)lens[i],
                                               rows.data() + (size_t)i * kMaxSeq, kMaxSeq);
        }))
        return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "tokenization ran out of memory");
    size_t p = 0;
    for (int32_t i = 0; i < n_texts; i++) {
        std::copy_n(rows.begin() + (int64_t)i * kMaxSeq, lengths[i], rows.begin() + (int64_t)p);
        p += (size_t)lengths[i];
        if (n_tokens) n_tokens[i] = lengths[i];
    }
    void *scratch = nullptr;
    TZH_TRY(tzh_ctx_scratch(ctx, p * 4, &scratch));
    TZH_HIP(hipMemcpyAsync(scratch, rows.data(), p * 4, hipMemcpyHostToDevice, ctx->stream));
    TZH_HIP(hipStreamSynchronize(ctx->stream));
    return tzh_arctic_forward_batch(m, outputs, (const uint32_t *)scratch, lengths.data(), n_texts, 0);
}
