// Safetensors weight files -> device tensors: the reference's SafetensorsFile
// (src/runtime/weights.ts:58-194) and the per-tensor upload of its model loader
// (src/model/loader.ts:134-162), with the float conversion done on the GPU.
//
// Format: an 8-byte little-endian header length H, H bytes of JSON
//   {"name": {"dtype": "BF16", "shape": [..], "data_offsets": [begin, end]}, ...,
//    "__metadata__": {"key": "value", ...}}
// then the data block; a tensor's bytes are data[begin, end) (row-major, little-endian).
// The header is parsed by a small recursive-descent JSON reader (strings with escapes, integers,
// arrays, objects, literals).  Every entry must have a known dtype, a shape and data offsets that
// lie inside the file and whose length is numel * element size.
//
// Loading streams the tensor's byte range through two pinned host chunks: while chunk i is being
// copied to the device, chunk i+1 is read from the file (by kReaders threads in parallel; one
// thread reads the page cache at ~14 GB/s, the host link carries ~57 GB/s).  A
// raw load copies straight into the destination; a converting load copies each chunk into a
// device staging slot and converts it from there into the destination (one kernel per chunk).
// Conversions (bit-exact):
//   BF16 -> F32  bits << 16                                      (weights.ts:157-165)
//   F16  -> F32  IEEE half -> float, NaN -> sign | 0x7fc00000     (weights.ts:28-56, 167-176)
//   F32 / widened value -> F16 or BF16: round to nearest even; NaN -> sign | canonical quiet NaN
//   (the reference only widens; narrowing is this library's addition for bf16/f16 compute).

#include <errno.h>
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "st_header.h"
#include "tsc_internal.h"

static_assert(tsc::kStNumDtypes == TSC_ST_F8_E5M2 + 1, "dtype codes of st_header.h match tsc.h");

namespace tsc {
namespace {

// ---------------------------------------------------------------------------------- convert
constexpr int kConvThreads = 256;

template <int SRC>
__device__ __forceinline__ float widen(uint32_t v) {
  if (SRC == TSC_ST_F32) return __uint_as_float(v);
  if (SRC == TSC_ST_BF16) return __uint_as_float(v << 16);
  // F16: exact widening (half subnormals are normal floats); NaN canonical with its sign
  const float x = (float)__builtin_bit_cast(_Float16, (uint16_t)v);
  return x != x ? __uint_as_float(((v & 0x8000u) << 16) | 0x7fc00000u) : x;
}

__device__ __forceinline__ uint16_t narrow_bf16(float x) {
  const uint32_t u = __float_as_uint(x);
  if (x != x) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint16_t narrow_f16(float x) {
  if (x != x) return (uint16_t)(((__float_as_uint(x) >> 16) & 0x8000u) | 0x7e00u);
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

template <int SRC, int DST>
__global__ void __launch_bounds__(kConvThreads)
    convert_kernel(const void* __restrict__ src, void* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kConvThreads;
  for (int64_t i = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; i < n; i += stride) {
    const uint32_t v = SRC == TSC_ST_F32 ? ((const uint32_t*)src)[i] : ((const uint16_t*)src)[i];
    const float x = widen<SRC>(v);
    if (DST == TSC_F32) ((float*)dst)[i] = x;
    else if (DST == TSC_BF16) ((uint16_t*)dst)[i] = narrow_bf16(x);
    else ((uint16_t*)dst)[i] = narrow_f16(x);
  }
}

template <int SRC>
void convert_to(hipStream_t s, int dst_dtype, const void* src, void* dst, int64_t n) {
  const unsigned grid = (unsigned)std::min<int64_t>((n + kConvThreads - 1) / kConvThreads, 4096);
  if (dst_dtype == TSC_F32) convert_kernel<SRC, TSC_F32><<<grid, kConvThreads, 0, s>>>(src, dst, n);
  else if (dst_dtype == TSC_BF16) convert_kernel<SRC, TSC_BF16><<<grid, kConvThreads, 0, s>>>(src, dst, n);
  else convert_kernel<SRC, TSC_F16><<<grid, kConvThreads, 0, s>>>(src, dst, n);
}

void convert(hipStream_t s, int src_dtype, int dst_dtype, const void* src, void* dst, int64_t n) {
  if (src_dtype == TSC_ST_F32) convert_to<TSC_ST_F32>(s, dst_dtype, src, dst, n);
  else if (src_dtype == TSC_ST_BF16) convert_to<TSC_ST_BF16>(s, dst_dtype, src, dst, n);
  else convert_to<TSC_ST_F16>(s, dst_dtype, src, dst, n);
}

// ---------------------------------------------------------------------------------- streaming
constexpr size_t kChunk = (size_t)16 << 20;  // bytes per pinned chunk (a multiple of 8)
constexpr int kReaders = 8;                  // threads reading one chunk from the file

// Process-wide pool of kReaders - 1 file readers; the calling thread reads the first slice.
// One chunk at a time (calls from several host threads take turns).
class ReadPool {
 public:
  bool read(int fd, int64_t off, size_t len, char* dst) {
    std::lock_guard<std::mutex> one(call_);
    const size_t slice = ((len + kReaders - 1) / kReaders + 4095) / 4096 * 4096;
    if (len < ((size_t)2 << 20)) return read_range(fd, off, dst, 0, len);
    {
      std::lock_guard<std::mutex> g(m_);
      if (threads_.empty())
        for (int t = 1; t < kReaders; ++t) threads_.emplace_back([this, t] { worker(t); });
      fd_ = fd;
      off_ = off;
      len_ = len;
      dst_ = dst;
      slice_ = slice;
      pending_ = kReaders - 1;
      ok_ = true;
      ++generation_;
    }
    cv_.notify_all();
    bool ok = read_range(fd, off, dst, 0, std::min(len, slice));
    std::unique_lock<std::mutex> g(m_);
    done_.wait(g, [this] { return pending_ == 0; });
    return ok && ok_;
  }

 private:
  static bool read_range(int fd, int64_t off, char* dst, size_t b, size_t e) {
    while (b < e) {
      const ssize_t r = pread(fd, dst + b, e - b, (off_t)(off + (int64_t)b));
      if (r <= 0) return false;
      b += (size_t)r;
    }
    return true;
  }
  void worker(int t) {
    uint64_t seen = 0;
    for (;;) {
      int fd;
      int64_t off;
      size_t len, slice;
      char* dst;
      {
        std::unique_lock<std::mutex> g(m_);
        cv_.wait(g, [&] { return generation_ != seen; });
        seen = generation_;
        fd = fd_, off = off_, len = len_, slice = slice_, dst = dst_;
      }
      const size_t b = std::min(len, slice * t), e = std::min(len, slice * (t + 1));
      const bool ok = read_range(fd, off, dst, b, e);
      {
        std::lock_guard<std::mutex> g(m_);
        ok_ = ok_ && ok;
        if (--pending_ == 0) done_.notify_one();
      }
    }
  }
  std::mutex call_, m_;
  std::condition_variable cv_, done_;
  std::vector<std::thread> threads_;
  uint64_t generation_ = 0;
  int pending_ = 0;
  bool ok_ = true;
  int fd_ = -1;
  int64_t off_ = 0;
  size_t len_ = 0, slice_ = 0;
  char* dst_ = nullptr;
};

// The pool of this process.  A forked child (a data-loader worker, say) gets a pool of its own:
// the parent's reader threads do not exist there.  Pools are never destroyed; their idle threads
// end with the process.
ReadPool& read_pool() {
  static std::mutex m;
  static ReadPool* pool = nullptr;
  static pid_t owner = 0;
  std::lock_guard<std::mutex> g(m);
  if (!pool || owner != getpid()) {
    pool = new ReadPool();
    owner = getpid();
  }
  return *pool;
}

int staging(tsc_ctx* ctx) {
  for (int b = 0; b < 2; ++b) {
    if (ctx->st_pin[b]) continue;
    if (hipHostMalloc(&ctx->st_pin[b], kChunk) != hipSuccess) {
      (void)hipGetLastError();
      ctx->st_pin[b] = nullptr;
      return fail(TSC_ERR_OOM, "safetensors: cannot allocate %zu bytes of pinned staging", kChunk);
    }
    const int st = check_hip(hipEventCreateWithFlags(&ctx->st_ev[b], hipEventDisableTiming),
                             "safetensors event");
    if (st) {
      (void)hipHostFree(ctx->st_pin[b]);
      ctx->st_pin[b] = nullptr;
      ctx->st_ev[b] = nullptr;
      return st;
    }
  }
  return TSC_OK;
}

int copy_string(const std::string& s, char* buf, int32_t len, const char* what) {
  if (!buf || len <= (int32_t)s.size())
    return fail(TSC_ERR_INVALID, "safetensors: %s needs a buffer of %zu bytes", what, s.size() + 1);
  memcpy(buf, s.c_str(), s.size() + 1);
  return TSC_OK;
}

}  // namespace

void st_release(tsc_ctx* ctx) {
  for (int b = 0; b < 2; ++b) {
    if (ctx->st_ev[b]) (void)hipEventDestroy(ctx->st_ev[b]);
    if (ctx->st_pin[b]) (void)hipHostFree(ctx->st_pin[b]);
    ctx->st_ev[b] = nullptr;
    ctx->st_pin[b] = nullptr;
    ctx->st_pending[b] = false;
  }
}

int st_open(const char* path, tsc_st** out) {
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(TSC_ERR_INVALID, "safetensors: cannot open %s: %s", path, strerror(errno));
  tsc_st* f = new tsc_st();
  f->fd = fd;
  const off_t size = lseek(fd, 0, SEEK_END);
  uint8_t lenb[8];
  int st = TSC_OK;
  if (size < 8 || pread(fd, lenb, 8, 0) != 8) {
    st = fail(TSC_ERR_INVALID, "safetensors: %s is shorter than its 8-byte header length", path);
  } else {
    uint64_t h = 0;
    for (int k = 7; k >= 0; --k) h = (h << 8) | lenb[k];
    if (h > (uint64_t)size - 8 || h > ((uint64_t)100 << 20)) {
      st = fail(TSC_ERR_INVALID, "safetensors: header length %llu does not fit %s",
                (unsigned long long)h, path);
    } else {
      std::string text(h, '\0');
      if (h && pread(fd, &text[0], h, 8) != (ssize_t)h) {
        st = fail(TSC_ERR_INVALID, "safetensors: cannot read the header of %s", path);
      } else {
        f->data_begin = 8 + (int64_t)h;
        f->file_size = (int64_t)size;
        std::string err;
        if (!st_parse_header(f, text.data(), text.size(), &err))
          st = fail(TSC_ERR_INVALID, "safetensors header: %s", err.c_str());
      }
    }
  }
  if (st) {
    close(fd);
    delete f;
    return st;
  }
  *out = f;
  return TSC_OK;
}

void st_close(tsc_st* f) {
  if (f->fd >= 0) close(f->fd);
  delete f;
}

void st_counts(const tsc_st* f, int64_t* tensors, int64_t* metadata, int64_t* data_offset) {
  if (tensors) *tensors = (int64_t)f->names.size();
  if (metadata) *metadata = (int64_t)f->metadata.size();
  if (data_offset) *data_offset = f->data_begin;
}

int st_name(const tsc_st* f, int64_t i, char* buf, int32_t len) {
  if (i < 0 || i >= (int64_t)f->names.size())
    return fail(TSC_ERR_INVALID, "safetensors: tensor index %lld out of range", (long long)i);
  return copy_string(f->names[i], buf, len, "tensor name");
}

int st_metadata(const tsc_st* f, int64_t i, char* key, int32_t key_len, char* value,
                int32_t value_len) {
  if (i < 0 || i >= (int64_t)f->metadata.size())
    return fail(TSC_ERR_INVALID, "safetensors: metadata index %lld out of range", (long long)i);
  int st = copy_string(f->metadata[i].first, key, key_len, "metadata key");
  if (st) return st;
  return copy_string(f->metadata[i].second, value, value_len, "metadata value");
}

int st_info(const tsc_st* f, const char* name, int32_t* dtype, int32_t* ndim, int64_t* shape,
            int32_t max_dims, int64_t* offsets) {
  auto it = f->index.find(name);
  if (it == f->index.end()) return fail(TSC_ERR_INVALID, "safetensors: no tensor named \"%s\"", name);
  const tsc_st::Entry& e = f->entries[it->second];
  if (shape && (int32_t)e.shape.size() > max_dims)
    return fail(TSC_ERR_INVALID, "safetensors: %s has %zu dims, the shape buffer holds %d", name,
                e.shape.size(), max_dims);
  if (dtype) *dtype = e.dtype;
  if (ndim) *ndim = (int32_t)e.shape.size();
  if (shape)
    for (size_t d = 0; d < e.shape.size(); ++d) shape[d] = e.shape[d];
  if (offsets) {
    offsets[0] = e.begin;
    offsets[1] = e.end;
  }
  return TSC_OK;
}

int st_load(tsc_ctx* ctx, const tsc_st* f, const char* name, int32_t out_dtype, void* dst) {
  auto it = f->index.find(name);
  if (it == f->index.end()) return fail(TSC_ERR_INVALID, "safetensors: no tensor named \"%s\"", name);
  const tsc_st::Entry& e = f->entries[it->second];
  const int64_t bytes = e.end - e.begin;
  const int src = e.dtype;
  const bool is_float = src == TSC_ST_F32 || src == TSC_ST_F16 || src == TSC_ST_BF16;
  const bool raw = out_dtype == TSC_ST_RAW || (is_float && out_dtype == src);
  if (!raw && out_dtype != TSC_F32 && out_dtype != TSC_F16 && out_dtype != TSC_BF16)
    return fail(TSC_ERR_INVALID, "safetensors: unknown output dtype %d", out_dtype);
  if (!raw && !is_float)
    return fail(TSC_ERR_UNSUPPORTED, "safetensors: %s is %s, not F32/F16/BF16; load it raw", name,
                st_dtype_name(src));
  if (bytes == 0) return TSC_OK;
  if (!dst) return fail(TSC_ERR_INVALID, "safetensors: null destination for %s", name);
  int st = staging(ctx);
  if (st) return st;
  const int src_size = st_dtype_size(src);
  const int dst_size = raw ? src_size : (out_dtype == TSC_F32 ? 4 : 2);
  char* dev_stage = nullptr;
  if (!raw) {
    void* ws;
    st = workspace(ctx, 2 * kChunk, &ws);
    if (st) return st;
    dev_stage = (char*)ws;
  }
  const int64_t file_off = f->data_begin + e.begin;
  // The two chunks alternate across calls too, so that the next tensor's first read overlaps
  // this tensor's last copy.
  for (int64_t done = 0; done < bytes; done += (int64_t)kChunk) {
    const int b = ctx->st_next;
    ctx->st_next ^= 1;
    const size_t len = (size_t)std::min<int64_t>(bytes - done, (int64_t)kChunk);
    // The pinned chunk is free once the copy that last read it has finished.
    if (ctx->st_pending[b]) {
      st = check_hip(hipEventSynchronize(ctx->st_ev[b]), "safetensors staging wait");
      if (st) return st;
      ctx->st_pending[b] = false;
    }
    if (!read_pool().read(f->fd, file_off + done, len, (char*)ctx->st_pin[b]))
      return fail(TSC_ERR_INVALID, "safetensors: short read of %s at byte %lld", name,
                  (long long)(file_off + done));
    char* target = raw ? (char*)dst + done : dev_stage + (size_t)b * kChunk;
    st = check_hip(hipMemcpyAsync(target, ctx->st_pin[b], len, hipMemcpyHostToDevice, ctx->stream),
                   "safetensors copy");
    if (st) return st;
    st = check_hip(hipEventRecord(ctx->st_ev[b], ctx->stream), "safetensors event record");
    if (st) return st;
    ctx->st_pending[b] = true;
    if (!raw) {
      ProfScope p(ctx, "st_convert");
      convert(ctx->stream, src, out_dtype, target, (char*)dst + done / src_size * dst_size,
              (int64_t)len / src_size);
      st = check_hip(hipGetLastError(), "safetensors convert");
      if (st) return st;
    }
  }
  return TSC_OK;
}

}  // namespace tsc
