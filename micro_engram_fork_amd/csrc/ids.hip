// The serving side of the Engram lookup path on gfx950: the per-step matrix of each scheduled
// token and the tokens before it, read by hash_prev in every engram layer, and the media mask.
//
// Reference (micro_engram_vllm/ids.py):
//   fill_engram_ids  10-59  out[t] = (token at t, token at t-1, ...), -1 where there is none;
//                           earlier tokens come from this step's input_ids when they are in the
//                           same chunk, otherwise from the request's history row
//   mask_media       62-70  media placeholder ids become -1 (missing history); keep[t] is false
//                           where the token itself is a media placeholder
//
// One thread per output row (token): it finds its request by binary search over
// query_start_loc, takes the chunk's first position, and fills max_order entries. Rows from
// num_tokens to num_tokens_padded are -1 (graph padding). The reference's lookback of the
// (max_order - 1) tokens before each chunk is indexed exactly as there: entry
// j = clamp(chunk_start - 1 - q, 0, max_order - 2) of the history positions chunk_start-1-j.
// With media ids given, the same launch applies the mask to the row it wrote and sets keep.
#include "me_common.h"

namespace me {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxMedia = 64;

struct Ptr {
    const void *p;
    int is64;
    __device__ __forceinline__ int64_t operator[](int64_t i) const {
        return is64 ? static_cast<const int64_t *>(p)[i]
                    : static_cast<int64_t>(static_cast<const int32_t *>(p)[i]);
    }
};

struct FillArgs {
    int32_t *out;
    int64_t out_stride;
    int max_order;
    Ptr ids, pos, map, qsl, hist;
    int64_t hist_rows, hist_len, hist_stride;
    int64_t num_reqs, num_tokens, num_padded;
    Ptr media;
    int n_media;
    uint8_t *keep;  // nullable
};

__device__ __forceinline__ bool in_media(int64_t v, const int64_t *s_media, int n_media) {
    bool hit = false;
    for (int i = 0; i < n_media; ++i) hit |= v == s_media[i];
    return hit;
}

__global__ __launch_bounds__(kThreads) void fill_ids_kernel(const FillArgs a) {
    __shared__ int64_t s_media[kMaxMedia];
    if (threadIdx.x < a.n_media) s_media[threadIdx.x] = a.media[threadIdx.x];
    __syncthreads();
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= a.num_padded) return;
    int32_t *row = a.out + t * a.out_stride;
    if (t >= a.num_tokens) {  // padding rows of a graph-sized batch: all -1
        for (int k = 0; k < a.max_order; ++k) row[k] = -1;
        if (a.keep != nullptr) a.keep[t] = in_media(-1, s_media, a.n_media) ? 0 : 1;
        return;
    }
    // request of this token: the last r with query_start_loc[r] <= t
    int64_t lo = 0, hi = a.num_reqs - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (a.qsl[mid] <= t) lo = mid; else hi = mid - 1;
    }
    int64_t begin = a.qsl[lo];
    begin = begin < a.num_tokens - 1 ? begin : a.num_tokens - 1;
    begin = begin < 0 ? 0 : begin;
    const int64_t start = a.pos[begin];  // first position run this step
    const int64_t state = a.map[lo];
    const bool state_ok = state >= 0 && state < a.hist_rows;
    const int64_t p = a.pos[t];
    int64_t first = a.ids[t];
    bool media0 = false;
    for (int k = 0; k < a.max_order; ++k) {
        int64_t v;
        if (k == 0) {
            v = first;
        } else {
            const int64_t q = p - k;
            if (q >= start) {
                const int64_t src = t - k;
                v = a.ids[src > 0 ? src : 0];
            } else {
                int64_t j = start - 1 - q;
                j = j < 0 ? 0 : (j > a.max_order - 2 ? a.max_order - 2 : j);
                const int64_t hp = start - 1 - j;
                v = (hp >= 0 && hp < a.hist_len && state_ok) ? a.hist[state * a.hist_stride + hp] : -1;
            }
        }
        if (a.n_media > 0 && in_media(v, s_media, a.n_media)) {
            if (k == 0) media0 = true;
            v = -1;
        }
        row[k] = static_cast<int32_t>(v);
    }
    if (a.keep != nullptr) a.keep[t] = media0 ? 0 : 1;
}

struct MaskArgs {
    Ptr ids;
    int64_t n, width, stride;
    int32_t *out;  // [n, width] contiguous
    uint8_t *keep;
    Ptr media;
    int n_media;
};

__global__ __launch_bounds__(kThreads) void mask_media_kernel(const MaskArgs a) {
    __shared__ int64_t s_media[kMaxMedia];
    if (threadIdx.x < a.n_media) s_media[threadIdx.x] = a.media[threadIdx.x];
    __syncthreads();
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= a.n) return;
    bool media0 = false;
    for (int64_t k = 0; k < a.width; ++k) {
        int64_t v = a.ids[t * a.stride + k];
        if (in_media(v, s_media, a.n_media)) {
            if (k == 0) media0 = true;
            v = -1;
        }
        a.out[t * a.width + k] = static_cast<int32_t>(v);
    }
    a.keep[t] = media0 ? 0 : 1;
}

int int_ptr(Ptr &p, const void *ptr, int dtype, const char *what) {
    if (dtype != ME_I32 && dtype != ME_I64) {
        set_error("%s dtype must be ME_I32 or ME_I64", what);
        return ME_ERR_INVALID;
    }
    p.p = ptr;
    p.is64 = dtype == ME_I64;
    return ME_OK;
}

}  // namespace
}  // namespace me

using namespace me;

#define ME_TRY(expr)                  \
    do {                              \
        const int _st = (expr);       \
        if (_st != ME_OK) return _st; \
    } while (0)

extern "C" int me_fill_engram_ids(int32_t *out, int64_t out_rows, int64_t out_row_stride,
                                  int32_t max_order, const void *input_ids, int ids_dtype,
                                  const void *positions, int pos_dtype, const void *idx_mapping,
                                  int map_dtype, const void *query_start_loc, int qsl_dtype,
                                  const void *all_token_ids, int hist_dtype, int64_t hist_rows,
                                  int64_t hist_len, int64_t hist_row_stride, int64_t num_reqs,
                                  int64_t num_tokens, int64_t num_tokens_padded,
                                  const void *media_ids, int media_dtype, int32_t n_media,
                                  uint8_t *keep_out, void *stream) {
    ME_CHECK_ARG(max_order >= 1 && max_order <= ME_MAX_ORDER, "max_order must be in [1, %d]",
                 ME_MAX_ORDER);
    ME_CHECK_ARG(num_tokens >= 0 && num_tokens_padded >= num_tokens,
                 "need 0 <= num_tokens <= num_tokens_padded");
    ME_CHECK_ARG(num_tokens_padded <= out_rows, "num_tokens_padded %lld exceeds the %lld rows of out",
                 (long long)num_tokens_padded, (long long)out_rows);
    ME_CHECK_ARG(out_row_stride >= max_order, "out row stride %lld < max_order %d",
                 (long long)out_row_stride, max_order);
    ME_CHECK_ARG(num_tokens_padded < (int64_t{1} << 31), "too many tokens");
    ME_CHECK_ARG(n_media >= 0 && n_media <= kMaxMedia, "n_media must be in [0, %d]", kMaxMedia);
    ME_CHECK_ARG(num_tokens == 0 || num_reqs >= 1, "num_tokens > 0 needs num_reqs >= 1");
    FillArgs a{};
    a.out = out;
    a.out_stride = out_row_stride;
    a.max_order = max_order;
    a.num_reqs = num_reqs;
    a.num_tokens = num_tokens;
    a.num_padded = num_tokens_padded;
    a.n_media = n_media;
    a.keep = keep_out;
    if (num_tokens > 0) {
        ME_CHECK_ARG(out && input_ids && positions && idx_mapping && query_start_loc && all_token_ids,
                     "null tensor pointer");
        ME_CHECK_ARG(hist_rows >= 1 && hist_len >= 1 && hist_row_stride >= hist_len,
                     "bad all_token_ids shape");
        ME_TRY(int_ptr(a.ids, input_ids, ids_dtype, "input_ids"));
        ME_TRY(int_ptr(a.pos, positions, pos_dtype, "positions"));
        ME_TRY(int_ptr(a.map, idx_mapping, map_dtype, "idx_mapping"));
        ME_TRY(int_ptr(a.qsl, query_start_loc, qsl_dtype, "query_start_loc"));
        ME_TRY(int_ptr(a.hist, all_token_ids, hist_dtype, "all_token_ids"));
        a.hist_rows = hist_rows;
        a.hist_len = hist_len;
        a.hist_stride = hist_row_stride;
    } else {
        ME_CHECK_ARG(out != nullptr || num_tokens_padded == 0, "out is null");
    }
    if (n_media > 0) {
        ME_CHECK_ARG(media_ids != nullptr, "media_ids is null");
        ME_TRY(int_ptr(a.media, media_ids, media_dtype, "media_ids"));
    }
    if (num_tokens_padded == 0) return ME_OK;
    const dim3 grid(static_cast<unsigned>(ceil_div(num_tokens_padded, kThreads)));
    hipLaunchKernelGGL(fill_ids_kernel, grid, dim3(kThreads), 0, as_stream(stream), a);
    return check_launch("me_fill_engram_ids");
}

extern "C" int me_mask_media(const void *ids, int ids_dtype, int64_t n, int64_t width,
                             int64_t row_stride, const void *media_ids, int media_dtype,
                             int32_t n_media, int32_t *ids_out, uint8_t *keep_out, void *stream) {
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31) && width >= 1, "bad shape");
    ME_CHECK_ARG(row_stride >= width, "row_stride < width");
    ME_CHECK_ARG(n_media >= 0 && n_media <= kMaxMedia, "n_media must be in [0, %d]", kMaxMedia);
    if (n == 0) return ME_OK;
    ME_CHECK_ARG(ids && ids_out && keep_out, "null tensor pointer");
    MaskArgs a{};
    ME_TRY(int_ptr(a.ids, ids, ids_dtype, "ids"));
    a.n = n;
    a.width = width;
    a.stride = row_stride;
    a.out = ids_out;
    a.keep = keep_out;
    a.n_media = n_media;
    if (n_media > 0) {
        ME_CHECK_ARG(media_ids != nullptr, "media_ids is null");
        ME_TRY(int_ptr(a.media, media_ids, media_dtype, "media_ids"));
    }
    const dim3 grid(static_cast<unsigned>(ceil_div(n, kThreads)));
    hipLaunchKernelGGL(mask_media_kernel, grid, dim3(kThreads), 0, as_stream(stream), a);
    return check_launch("me_mask_media");
}
