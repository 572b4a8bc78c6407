// C-ABI implementation of libgustann_hip.so (declared in include/gustann.h).
//
// Host orchestration of the in-memory search path: the GustANN facade and the
// PURE_MEM executor of the reference (src/ssd_search.cu, src/pure_mem.cu),
// the PQ loader/uploader (src/pq_search.cu) and the nav-graph loader
// (src/nav_graph.cu), with device residency, validation and error codes in
// place of the reference's exit()/abort()/throw.
#include "../../include/gustann.h"

#include <fcntl.h>
#include <linux/io_uring.h>
#include <sys/mman.h>
#include <sys/syscall.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <functional>
#include <memory>
#include <mutex>
#include <numeric>
#include <random>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "formats.hpp"
#include "gann_build.hpp"
#include "gann_kernels.hpp"
#include "gann_knn.hpp"

namespace {

thread_local std::string g_err;

struct Error {
  int code;
  std::string msg;
};

#define GANN_HIP(expr)                                                                         \
  do {                                                                                         \
    hipError_t e_ = (expr);                                                                    \
    if (e_ != hipSuccess)                                                                      \
      throw Error{e_ == hipErrorOutOfMemory ? GANN_ERR_NOMEM : GANN_ERR_HIP,                   \
                  std::string(#expr) + ": " + hipGetErrorString(e_)};                          \
  } while (0)

template <class F>
int guarded(F&& f) {
  try {
    f();
    return GANN_OK;
  } catch (const Error& e) {
    g_err = e.msg;
    return e.code;
  } catch (const std::bad_alloc&) {
    g_err = "host allocation failed";
    return GANN_ERR_NOMEM;
  } catch (const std::exception& e) {
    g_err = e.what();
    return GANN_ERR_INVALID;
  } catch (...) {
    g_err = "unknown error";
    return GANN_ERR_INVALID;
  }
}

[[noreturn]] void raise(int code, const std::string& msg) { throw Error{code, msg}; }

// Device allocation owned by RAII.
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { release(); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  void ensure(size_t n) {
    if (n <= bytes && p) return;
    release();
    GANN_HIP(hipMalloc(&p, n ? n : 1));
    bytes = n;
  }
  template <class T>
  T* as() const {
    return reinterpret_cast<T*>(p);
  }
};

struct PinnedBuf {
  void* p = nullptr;
  size_t bytes = 0;
  PinnedBuf() = default;
  PinnedBuf(const PinnedBuf&) = delete;
  PinnedBuf& operator=(const PinnedBuf&) = delete;
  ~PinnedBuf() {
    if (p) (void)hipHostFree(p);
  }
  void alloc(size_t n, unsigned extra_flags = 0) {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    GANN_HIP(hipHostMalloc(&p, n ? n : 1, hipHostMallocMapped | hipHostMallocPortable | extra_flags));
    bytes = n;
  }
  void ensure(size_t n, unsigned extra_flags = 0) {
    if (!p || n > bytes) alloc(n, extra_flags);
  }
};

void upload(DevBuf& d, const void* src, size_t bytes) {
  d.ensure(bytes);
  if (bytes) GANN_HIP(hipMemcpy(d.p, src, bytes, hipMemcpyHostToDevice));
}

double now_s() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

unsigned host_threads() {
  unsigned t = std::thread::hardware_concurrency();
  return t == 0 ? 4 : std::min(t, 16u);
}

// Checks every node record of a block of pages: deg <= R, neighbour ids
// < num_pts, no id twice in one list.  The reference does not check
// (src/impl/pure_mem.cuh:288-301 indexes with whatever the file holds); the
// kernels index the code table with these ids, so they are validated once here.
void validate_pages(const gann::DiskLayout& L, const uint8_t* pages, int64_t first_page,
                    int64_t npages, std::atomic<int64_t>* bad_node) {
  int64_t u0 = first_page * L.nodes_per_page;
  int64_t u1 = std::min(L.num_pts, (first_page + npages) * L.nodes_per_page);
  unsigned nt = host_threads();
  std::vector<std::thread> th;
  for (unsigned t = 0; t < nt; ++t) {
    th.emplace_back([&, t] {
      std::vector<uint32_t> tmp((size_t)L.max_m);
      for (int64_t u = u0 + t; u < u1; u += nt) {
        if (bad_node->load(std::memory_order_relaxed) >= 0) return;
        const uint8_t* rec = pages + (u / L.nodes_per_page - first_page) * gann::kSectorBytes +
                             (u % L.nodes_per_page) * L.node_len;
        int32_t deg;
        std::memcpy(&deg, rec + L.data_len, 4);
        bool ok = deg >= 0 && deg <= L.max_m;
        if (ok) {
          std::memcpy(tmp.data(), rec + L.data_len + 4, (size_t)deg * 4);
          for (int32_t j = 0; j < deg && ok; ++j) ok = tmp[(size_t)j] < (uint64_t)L.num_pts;
          if (ok) {
            std::sort(tmp.begin(), tmp.begin() + deg);
            ok = std::adjacent_find(tmp.begin(), tmp.begin() + deg) == tmp.begin() + deg;
          }
        }
        if (!ok) {
          int64_t expect = -1;
          bad_node->compare_exchange_strong(expect, u);
          return;
        }
      }
    });
  }
  for (auto& x : th) x.join();
}

}  // namespace

// ---------------------------------------------------------------- PQ object

struct gann_pq {
  int device = 0;
  hipStream_t stream = nullptr;
  gann::PQDev dev{};
  DevBuf pivots, pivots_t, centroid, chunk_off, codes, piv_cb;
  bool codes_borrowed = false;
  // scratch of the host-pointer entry points
  DevBuf q, ids, out;

  ~gann_pq() {
    if (stream) {
      (void)hipSetDevice(device);
      (void)hipStreamDestroy(stream);
    }
  }

  // Uploads pivots (transposed to [dim][256] as src/pq_search.cu:88-93),
  // centroid and chunk offsets.
  void upload_static(const float* pivots, const float* c, const int32_t* off, int dim, int M) {
    std::vector<float> pt((size_t)dim * gann::kNumPivots);
    for (int i = 0; i < gann::kNumPivots; ++i)
      for (int j = 0; j < dim; ++j) pt[(size_t)j * gann::kNumPivots + i] = pivots[(size_t)i * dim + j];
    upload(pivots_t, pt.data(), pt.size() * 4);
    upload(this->pivots, pivots, (size_t)gann::kNumPivots * dim * 4);
    std::vector<uint8_t> cb(gann::search_cb_pivot_bytes(dim));
    gann::search_cb_pivot_layout(pivots, dim, cb.data());
    upload(piv_cb, cb.data(), cb.size());
    upload(centroid, c, (size_t)dim * 4);
    upload(chunk_off, off, (size_t)(M + 1) * 4);
    dev.dim = dim;
    dev.M = M;
    // uniform chunks [m*w, (m+1)*w) select the unrolled LUT build
    int w = dim % M == 0 ? dim / M : 0;
    for (int m = 0; m <= M && w; ++m)
      if (off[m] != m * w) w = 0;
    dev.chunk_w = w;
    dev.pivots = this->pivots.as<float>();
    dev.pivots_t = pivots_t.as<float>();
    dev.centroid = centroid.as<float>();
    dev.chunk_off = chunk_off.as<int32_t>();
    dev.piv_cb = piv_cb.as<uint8_t>();
  }
};

namespace {

void check_chunks(const int32_t* off, int dim, int M) {
  if (M < 1 || dim < 1) raise(GANN_ERR_INVALID, "pq: need dim >= 1 and num_chunks >= 1");
  if (off[0] != 0 || off[M] != dim)
    raise(GANN_ERR_FORMAT, "pq chunk offsets must start at 0 and end at dim");
  for (int m = 0; m < M; ++m)
    if (off[m + 1] < off[m]) raise(GANN_ERR_FORMAT, "pq chunk offsets must be non-decreasing");
}

void check_lds(size_t bytes, int device, const char* what) {
  int lim = 0;
  GANN_HIP(hipDeviceGetAttribute(&lim, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
  if (bytes > (size_t)lim)
    raise(GANN_ERR_UNSUPPORTED, std::string(what) + ": LDS footprint " + std::to_string(bytes) +
                                    " B exceeds the device limit " + std::to_string(lim) + " B");
}

}  // namespace

// ---------------------------------------------------------------- handle

struct gann_handle {
  int device = 0;
  int num_cus = 0;
  size_t lds_limit = 0;
  int dtype = 0;
  int placement = GANN_PLACEMENT_HBM;
  hipStream_t stream = nullptr;
  gann::DiskLayout layout;
  gann_pq pq;
  // pages: HBM copy or pinned host memory
  DevBuf pages_dev;
  PinnedBuf pages_host;
  std::string index_path;          // page source of the page-fetch mode without host pages
  PinnedBuf slots, state_host;     // page-fetch mode: one page per query, state readback
  gann::IndexDev ix{};
  // pivot graph
  bool has_nav = false;
  gann::NavHost nav_host_meta;  // sizes only (data vectors released after upload)
  DevBuf nav_data, nav_graph, nav_map;
  gann::NavDev nav{};
  // per-call scratch
  DevBuf q, entries, local, nns, dists, found, nexp, nadc, counters, qs;
  DevBuf entry_dist, order;  // the fused kernels' query order (run_entries)
  DevBuf luts, lists, state;
  PinnedBuf counter_host;
  // this device's copy of the fixed scratch of gann_search_device_noalloc
  void* noalloc_scratch = nullptr;

  ~gann_handle() {
    if (stream) {
      (void)hipSetDevice(device);
      (void)hipStreamDestroy(stream);
    }
  }
};

namespace {

void open_handle(const gann_config* cfg, gann_handle* h) {
  if (!cfg || !cfg->index_file || !cfg->pq_prefix || !*cfg->pq_prefix)
    raise(GANN_ERR_INVALID, "config needs index_file and pq_prefix (src/ssd_search.cu:59-67)");
  if (cfg->dtype != GANN_UINT8 && cfg->dtype != GANN_FLOAT) raise(GANN_ERR_INVALID, "unknown dtype");
  if (cfg->placement != GANN_PLACEMENT_HBM && cfg->placement != GANN_PLACEMENT_HOST_PINNED)
    raise(GANN_ERR_INVALID, "unknown placement");
  int ndev = 0;
  GANN_HIP(hipGetDeviceCount(&ndev));
  if (cfg->device_id < 0 || cfg->device_id >= ndev) raise(GANN_ERR_INVALID, "device_id out of range");
  h->device = cfg->device_id;
  h->dtype = cfg->dtype;
  h->placement = cfg->placement;
  GANN_HIP(hipSetDevice(h->device));
  {
    int cus = 0, lds = 0;
    GANN_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, h->device));
    GANN_HIP(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, h->device));
    h->num_cus = cus;
    h->lds_limit = (size_t)lds;
  }
  GANN_HIP(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking));
  GANN_HIP(gann::noalloc_scratch_setup(h->device, &h->noalloc_scratch));
  h->pq.device = h->device;
  GANN_HIP(hipStreamCreateWithFlags(&h->pq.stream, hipStreamNonBlocking));

  std::string err;
  const int64_t es = cfg->dtype == GANN_UINT8 ? 1 : 4;
  h->index_path = cfg->index_file;
  if (!gann::parse_disk_meta(cfg->index_file, es, &h->layout, &err))
    raise(err.rfind("cannot open", 0) == 0 ? GANN_ERR_IO : GANN_ERR_FORMAT, err);
  const gann::DiskLayout& L = h->layout;
  // The degree and neighbour ids follow the coordinates in each record and
  // are read as 32-bit words (src/impl/pure_mem.cuh:290-292), which needs a
  // 4-byte aligned coordinate block.
  if (L.data_len % 4 != 0)
    raise(GANN_ERR_UNSUPPORTED, "coordinate bytes per record must be a multiple of 4");

  // PQ (src/ssd_search.cu:59-67, src/pq_search.cu:56-121)
  {
    gann::PQHost pqh;
    std::string pp = std::string(cfg->pq_prefix);
    if (!gann::read_pq(pp + "_pivots.bin", pp + "_compressed.bin", &pqh, true, &err))
      raise(err.rfind("cannot open", 0) == 0 ? GANN_ERR_IO : GANN_ERR_FORMAT, err);
    if (pqh.dim != L.dim) raise(GANN_ERR_FORMAT, "pq dim differs from the index dim");  // :124
    if (pqh.num_pts != L.num_pts)
      raise(GANN_ERR_FORMAT, "pq point count differs from the index");  // :125
    check_chunks(pqh.chunk_offsets.data(), pqh.dim, pqh.num_chunks);
    h->pq.upload_static(pqh.pivots.data(), pqh.centroid.data(), pqh.chunk_offsets.data(), pqh.dim,
                        pqh.num_chunks);
    upload(h->pq.codes, pqh.codes.data(), pqh.codes.size());
    h->pq.dev.codes = h->pq.codes.as<uint8_t>();
    h->pq.dev.num_pts = pqh.num_pts;
  }

  // pivot graph (src/ssd_search.cu:70-78, src/nav_graph.cu:41-100)
  if (cfg->nav_prefix && *cfg->nav_prefix) {
    gann::NavHost nh;
    if (!gann::read_nav(cfg->nav_prefix, es, &nh, &err))
      raise(err.rfind("cannot open", 0) == 0 ? GANN_ERR_IO : GANN_ERR_FORMAT, err);
    if (nh.dim != L.dim) raise(GANN_ERR_FORMAT, "nav_index.data dim differs from the index dim");
    upload(h->nav_data, nh.data.data(), nh.data.size());
    upload(h->nav_graph, nh.graph.data(), nh.graph.size() * 4);
    upload(h->nav_map, nh.mapping.data(), nh.mapping.size() * 4);
    h->has_nav = true;
    h->nav_host_meta.num_node = nh.num_node;
    h->nav_host_meta.dim = nh.dim;
    h->nav_host_meta.max_m = nh.max_m;
    h->nav_host_meta.start = nh.start;
    h->nav = gann::NavDev{h->nav_data.as<uint8_t>(), h->nav_graph.as<int32_t>(),
                          h->nav_map.as<int32_t>(), nh.num_node, nh.max_m, nh.start};
  }

  // pages (src/pure_mem.cu:45-69): read through a pinned staging ring into
  // HBM, or keep them in pinned host memory for the zero-copy placement.
  const int64_t total = L.num_pages * gann::kSectorBytes;
  std::atomic<int64_t> bad{-1};
  gann::File f(cfg->index_file, "rb");
  if (!f || !f.seek(gann::kSectorBytes)) raise(GANN_ERR_IO, "cannot read index pages");
  if (cfg->placement == GANN_PLACEMENT_HOST_PINNED) {
    h->pages_host.alloc((size_t)total);
    const int64_t chunk_pages = 65536;  // 256 MiB
    for (int64_t p0 = 0; p0 < L.num_pages; p0 += chunk_pages) {
      int64_t np = std::min(chunk_pages, L.num_pages - p0);
      uint8_t* dst = (uint8_t*)h->pages_host.p + p0 * gann::kSectorBytes;
      if (!f.read(dst, (size_t)(np * gann::kSectorBytes))) raise(GANN_ERR_FORMAT, "short read of index pages");
      validate_pages(L, dst, p0, np, &bad);
    }
    void* dptr = nullptr;
    GANN_HIP(hipHostGetDevicePointer(&dptr, h->pages_host.p, 0));
    h->ix.pages = (const uint8_t*)dptr;
  } else {
    h->pages_dev.ensure((size_t)total);
    const int64_t chunk_pages = 16384;  // 64 MiB per staging buffer
    PinnedBuf stage[2];
    stage[0].alloc((size_t)(chunk_pages * gann::kSectorBytes));
    stage[1].alloc((size_t)(chunk_pages * gann::kSectorBytes));
    hipEvent_t done[2];
    bool recorded[2] = {false, false};
    GANN_HIP(hipEventCreate(&done[0]));
    GANN_HIP(hipEventCreate(&done[1]));
    int k = 0;
    for (int64_t p0 = 0; p0 < L.num_pages; p0 += chunk_pages, k ^= 1) {
      int64_t np = std::min(chunk_pages, L.num_pages - p0);
      if (recorded[k]) GANN_HIP(hipEventSynchronize(done[k]));
      uint8_t* buf = (uint8_t*)stage[k].p;
      if (!f.read(buf, (size_t)(np * gann::kSectorBytes))) raise(GANN_ERR_FORMAT, "short read of index pages");
      validate_pages(L, buf, p0, np, &bad);
      GANN_HIP(hipMemcpyAsync((uint8_t*)h->pages_dev.p + p0 * gann::kSectorBytes, buf,
                              (size_t)(np * gann::kSectorBytes), hipMemcpyHostToDevice, h->stream));
      GANN_HIP(hipEventRecord(done[k], h->stream));
      recorded[k] = true;
    }
    GANN_HIP(hipStreamSynchronize(h->stream));
    (void)hipEventDestroy(done[0]);
    (void)hipEventDestroy(done[1]);
    h->ix.pages = h->pages_dev.as<uint8_t>();
  }
  if (bad.load() >= 0)
    raise(GANN_ERR_FORMAT, "node record " + std::to_string(bad.load()) +
                               ": degree > R, neighbour id out of range or repeated");
  h->ix.nodes_per_page = L.nodes_per_page;
  h->ix.node_len = L.node_len;
  h->ix.data_len = L.data_len;
  h->ix.num_pts = L.num_pts;
  h->ix.medoid = L.medoid;
  h->ix.R = (int32_t)L.max_m;
  h->ix.dim = (int32_t)L.dim;
  gann::set_page_divisor(h->ix);
  h->counter_host.alloc(64);
}

void validate_search(const gann_handle* h, int32_t nq, int32_t topk, int32_t L, int32_t beam) {
  if (nq < 0) raise(GANN_ERR_INVALID, "nq must be >= 0");
  if (topk < 1) raise(GANN_ERR_INVALID, "topk must be >= 1");
  if (L < topk) raise(GANN_ERR_INVALID, "L (ef_search) must be >= topk (bin/search_disk.cpp:189-192)");
  if (beam < 1) raise(GANN_ERR_INVALID, "beam_width must be >= 1 (1 = the reference's one node per iteration)");
  if (beam > gann::max_beam_width())
    raise(GANN_ERR_UNSUPPORTED, "beam_width must be in [1, " + std::to_string(gann::max_beam_width()) +
                                    "] (1 = the reference's one node per iteration)");
  if (h->layout.max_m > 128)
    raise(GANN_ERR_UNSUPPORTED, "graph degree R > 128 is not supported (two 64-neighbour blocks per expansion)");
}

// Entry selection (src/pure_mem.cu:104-124): nav kernel + on-device
// translation, or the medoid.
void run_entries(gann_handle* h, const float* q_dev, int32_t nq, int32_t* entries, int32_t* local,
                 int32_t* fallback, hipStream_t s) {
  if (h->has_nav) {
    GANN_HIP(gann::launch_fill_i32(fallback, 1, 0, s));
    GANN_HIP(gann::launch_nav_entry(h->nav, h->dtype, h->layout.medoid, h->layout.num_pts,
                                    (int)h->layout.dim, q_dev, nq, entries, local, fallback, s));
  } else {
    GANN_HIP(gann::launch_fill_i32(entries, nq, (int32_t)h->layout.medoid, s));
    if (local) GANN_HIP(gann::launch_fill_i32(local, nq, -1, s));
    GANN_HIP(gann::launch_fill_i32(fallback, 1, 0, s));
  }
}

// Copies page `page` of the index (0-based, after the header sector) to dst:
// from the host page image when the handle has one, else from the file.
struct PageSource {
  const uint8_t* mem = nullptr;
  int fd = -1;
  ~PageSource() {
    if (fd >= 0) ::close(fd);
  }
  void open_for(const gann_handle* h) {
    mem = (const uint8_t*)h->pages_host.p;
    if (!mem) {
      fd = ::open(h->index_path.c_str(), O_RDONLY);
      if (fd < 0) raise(GANN_ERR_IO, "cannot open " + h->index_path + " for page reads");
    }
  }
  // Node u's record, into its place in the 4096-byte slot of its page (the
  // loaders move whole pages; the kernel reads only the record, so only those
  // bytes are copied).
  void read_record(int64_t u, int64_t npp, int64_t node_len, uint8_t* slot) const {
    const int64_t page = u / npp, off = (u % npp) * node_len;
    if (mem) {
      std::memcpy(slot + off, mem + page * gann::kSectorBytes + off, (size_t)node_len);
      return;
    }
    const off_t pos = (off_t)((page + 1) * gann::kSectorBytes + off);
    size_t got = 0;
    while (got < (size_t)node_len) {
      const ssize_t r = ::pread(fd, slot + off + got, (size_t)node_len - got, pos + (off_t)got);
      if (r <= 0) raise(GANN_ERR_IO, "short page read from " + path);
      got += (size_t)r;
    }
  }
  std::string path;
};

// Whole-page reads through io_uring, driven by its system calls (the ring
// set-up and the submission / completion protocol of the io_uring ABI; the
// role of src/io/io_uring.cpp's IoUringLoader, which uses liburing): page
// reads of 4096 bytes at queue depth up to `depth`, all of a batch reaped
// before read_pages returns.
class UringReader {
 public:
  UringReader() = default;
  UringReader(const UringReader&) = delete;
  UringReader& operator=(const UringReader&) = delete;
  ~UringReader() {
    if (sqes_) ::munmap(sqes_, sqe_len_);
    if (cq_map_ && cq_map_ != sq_map_) ::munmap(cq_map_, cq_len_);
    if (sq_map_) ::munmap(sq_map_, sq_len_);
    if (rfd_ >= 0) ::close(rfd_);
  }
  // false (errno set) when the kernel refuses io_uring
  bool init(unsigned depth) {
    io_uring_params p;
    std::memset(&p, 0, sizeof p);
    rfd_ = (int)::syscall(__NR_io_uring_setup, depth, &p);
    if (rfd_ < 0) return false;
    entries_ = p.sq_entries;
    sq_len_ = p.sq_off.array + p.sq_entries * sizeof(unsigned);
    cq_len_ = p.cq_off.cqes + p.cq_entries * sizeof(io_uring_cqe);
    const bool single = (p.features & IORING_FEAT_SINGLE_MMAP) != 0;
    if (single) sq_len_ = cq_len_ = std::max(sq_len_, cq_len_);
    sq_map_ = map(sq_len_, IORING_OFF_SQ_RING);
    cq_map_ = single ? sq_map_ : map(cq_len_, IORING_OFF_CQ_RING);
    sqe_len_ = p.sq_entries * sizeof(io_uring_sqe);
    sqes_ = (io_uring_sqe*)map(sqe_len_, IORING_OFF_SQES);
    if (!sq_map_ || !cq_map_ || !sqes_) return false;
    char* sq = (char*)sq_map_;
    char* cq = (char*)cq_map_;
    sq_head_ = (unsigned*)(sq + p.sq_off.head);
    sq_tail_ = (unsigned*)(sq + p.sq_off.tail);
    sq_mask_ = *(unsigned*)(sq + p.sq_off.ring_mask);
    sq_array_ = (unsigned*)(sq + p.sq_off.array);
    cq_head_ = (unsigned*)(cq + p.cq_off.head);
    cq_tail_ = (unsigned*)(cq + p.cq_off.tail);
    cq_mask_ = *(unsigned*)(cq + p.cq_off.ring_mask);
    cqes_ = (io_uring_cqe*)(cq + p.cq_off.cqes);
    return true;
  }
  // dst[i] <- the 4096 bytes at file offset off[i]; bytes past the end of
  // the file read as zero.  Returns an error message, or "" on success.
  std::string read_pages(int fd, const std::vector<std::pair<uint8_t*, off_t>>& reqs) {
    const size_t n = reqs.size();
    size_t next = 0, done = 0, inflight = 0;
    std::string err;
    while (done < n) {
      unsigned tail = *sq_tail_;
      const unsigned head = __atomic_load_n(sq_head_, __ATOMIC_ACQUIRE);
      unsigned to_submit = 0;
      while (next < n && inflight < entries_ && tail - head < entries_) {
        const unsigned idx = tail & sq_mask_;
        io_uring_sqe* e = &sqes_[idx];
        std::memset(e, 0, sizeof *e);
        e->opcode = IORING_OP_READ;
        e->fd = fd;
        e->addr = (uint64_t)(uintptr_t)reqs[next].first;
        e->len = (uint32_t)gann::kSectorBytes;
        e->off = (uint64_t)reqs[next].second;
        e->user_data = (uint64_t)next;
        sq_array_[idx] = idx;
        ++tail;
        ++next;
        ++inflight;
        ++to_submit;
      }
      __atomic_store_n(sq_tail_, tail, __ATOMIC_RELEASE);
      const long r = ::syscall(__NR_io_uring_enter, rfd_, to_submit, 1u, IORING_ENTER_GETEVENTS, nullptr, 0);
      if (r < 0 && errno != EINTR) return std::string("io_uring_enter: ") + std::strerror(errno);
      unsigned ch = *cq_head_;
      const unsigned ct = __atomic_load_n(cq_tail_, __ATOMIC_ACQUIRE);
      for (; ch != ct; ++ch) {
        const io_uring_cqe& c = cqes_[ch & cq_mask_];
        const size_t i = (size_t)c.user_data;
        if (c.res < 0) {
          if (err.empty()) err = std::string("page read: ") + std::strerror(-c.res);
        } else if (i < n && c.res < (int)gann::kSectorBytes) {
          std::memset(reqs[i].first + c.res, 0, gann::kSectorBytes - (size_t)c.res);
        }
        ++done;
        --inflight;
      }
      __atomic_store_n(cq_head_, ch, __ATOMIC_RELEASE);
    }
    return err;
  }

 private:
  void* map(size_t len, off_t what) {
    void* m = ::mmap(nullptr, len, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, rfd_, what);
    return m == MAP_FAILED ? nullptr : m;
  }
  int rfd_ = -1;
  unsigned entries_ = 0, sq_mask_ = 0, cq_mask_ = 0;
  void *sq_map_ = nullptr, *cq_map_ = nullptr;
  size_t sq_len_ = 0, cq_len_ = 0, sqe_len_ = 0;
  unsigned *sq_head_ = nullptr, *sq_tail_ = nullptr, *sq_array_ = nullptr;
  unsigned *cq_head_ = nullptr, *cq_tail_ = nullptr;
  io_uring_sqe* sqes_ = nullptr;
  io_uring_cqe* cqes_ = nullptr;
};

// A fixed team of host threads that runs fn(t), t in [0, n), and waits; the
// calling thread is member 0.
class ThreadTeam {
 public:
  explicit ThreadTeam(int n) : n_(n) {
    for (int t = 1; t < n; ++t) th_.emplace_back([this, t] { loop(t); });
  }
  ThreadTeam(const ThreadTeam&) = delete;
  ThreadTeam& operator=(const ThreadTeam&) = delete;
  ~ThreadTeam() {
    {
      std::lock_guard<std::mutex> g(m_);
      stop_ = true;
      ++gen_;
    }
    cv_.notify_all();
    for (auto& t : th_) t.join();
  }
  void run(const std::function<void(int)>& fn) {
    {
      std::lock_guard<std::mutex> g(m_);
      fn_ = &fn;
      left_ = n_ - 1;
      ++gen_;
    }
    cv_.notify_all();
    fn(0);
    std::unique_lock<std::mutex> l(m_);
    done_.wait(l, [&] { return left_ == 0; });
  }

 private:
  void loop(int t) {
    int seen = 0;
    for (;;) {
      const std::function<void(int)>* f;
      {
        std::unique_lock<std::mutex> l(m_);
        cv_.wait(l, [&] { return gen_ != seen; });
        seen = gen_;
        if (stop_) return;
        f = fn_;
      }
      (*f)(t);
      std::lock_guard<std::mutex> g(m_);
      if (--left_ == 0) done_.notify_one();
    }
  }
  int n_;
  std::vector<std::thread> th_;
  std::mutex m_;
  std::condition_variable cv_, done_;
  const std::function<void(int)>* fn_ = nullptr;
  int left_ = 0, gen_ = 0;
  bool stop_ = false;
};

// Step-wise search with a page-fetch stage (the hybrid executor's round,
// src/hyd_task_runner.cu:126-275, with MemLoaderSync, src/io/mem_io.cpp:11-44):
// after each GPU round the host reads every query's next node, copies that
// node's record into its place in the query's 4096-byte page slot of a
// pinned, device-mapped buffer, and the next round reads it from the slot.  The kernels
// and therefore the results are those of GANN_MODE_STEPWISE.
void run_stepwise_paged(gann_handle* h, const float* q_dev, int32_t nq, int32_t topk, int32_t L,
                        const int32_t* entries, int32_t* nns, float* dists, int32_t* found,
                        int32_t* nexp, int32_t* nadc, hipStream_t s, bool uring) {
  const gann::DiskLayout& Ly = h->layout;
  h->luts.ensure((size_t)nq * h->pq.dev.M * gann::kNumPivots * 4);
  h->lists.ensure((size_t)nq * L * 8);
  const size_t sb = gann::step_state_bytes();
  h->state.ensure((size_t)nq * sb);
  h->counters.ensure(64);
  h->slots.ensure((size_t)nq * gann::kSectorBytes, hipHostMallocCoherent);
  h->state_host.ensure((size_t)nq * sb);
  void* slots_dev = nullptr;
  GANN_HIP(hipHostGetDevicePointer(&slots_dev, h->slots.p, 0));
  PageSource src;
  src.path = h->index_path;
  // io_uring: whole pages from the index file, O_DIRECT where the file
  // system takes it (the reference's loader opens with O_DIRECT), one ring
  // per host thread (the reference's one ring per context)
  const int nthreads = (int)std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
  std::vector<std::unique_ptr<UringReader>> rings;
  int ufd = -1;
  struct FdCloser {
    int& fd;
    ~FdCloser() {
      if (fd >= 0) ::close(fd);
    }
  } ufd_closer{ufd};
  std::vector<std::vector<std::pair<uint8_t*, off_t>>> reqs((size_t)nthreads);
  if (uring) {
    ufd = ::open(h->index_path.c_str(), O_RDONLY | O_DIRECT);
    if (ufd < 0) ufd = ::open(h->index_path.c_str(), O_RDONLY);
    if (ufd < 0) raise(GANN_ERR_IO, "cannot open " + h->index_path + " for page reads");
    for (int t = 0; t < nthreads; ++t) {
      rings.emplace_back(new UringReader());
      if (!rings.back()->init(1024))
        raise(GANN_ERR_UNSUPPORTED, std::string("io_uring is not available: ") + std::strerror(errno));
    }
    // a file system that refuses O_DIRECT reads fails the first one: read
    // through the page cache then
    reqs[0].assign(1, {(uint8_t*)h->slots.p, (off_t)0});
    if (!rings[0]->read_pages(ufd, reqs[0]).empty()) {
      ::close(ufd);
      ufd = ::open(h->index_path.c_str(), O_RDONLY);
      if (ufd < 0) raise(GANN_ERR_IO, "cannot open " + h->index_path + " for page reads");
    }
  } else {
    src.open_for(h);
  }
  GANN_HIP(gann::launch_step_init(h->pq.dev, q_dev, nq, entries, h->luts.as<float>(), h->state.p, s));
  int32_t* active = h->counters.as<int32_t>() + 1;
  GANN_HIP(gann::launch_fill_i32(active, 1, nq, s));
  ThreadTeam team(nthreads);
  std::vector<int32_t> req((size_t)nq);
  const int64_t max_rounds = Ly.num_pts + 2;
  for (int64_t r = 0; r < max_rounds; ++r) {
    GANN_HIP(hipMemcpyAsync(h->state_host.p, h->state.p, (size_t)nq * sb, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipStreamSynchronize(s));
    int64_t n_active = 0;
    for (int32_t j = 0; j < nq; ++j) {
      req[(size_t)j] = gann::step_state_node(h->state_host.p, j);
      if (req[(size_t)j] >= 0) {
        if (req[(size_t)j] >= Ly.num_pts) raise(GANN_ERR_FORMAT, "request outside the index");
        ++n_active;
      }
    }
    if (n_active == 0) break;
    // submit_task: every active query's page (io_uring) or record into its slot
    if (uring) {
      std::vector<std::string> errs((size_t)nthreads);
      team.run([&](int t) {
        try {
          auto& rq = reqs[(size_t)t];
          rq.clear();
          for (int32_t j = t; j < nq; j += nthreads)
            if (req[(size_t)j] >= 0)
              rq.emplace_back((uint8_t*)h->slots.p + (size_t)j * gann::kSectorBytes,
                              (off_t)((req[(size_t)j] / Ly.nodes_per_page + 1) * gann::kSectorBytes));
          errs[(size_t)t] = rings[(size_t)t]->read_pages(ufd, rq);
        } catch (...) {
          errs[(size_t)t] = "page read request failed";
        }
      });
      for (const std::string& e : errs)
        if (!e.empty()) raise(GANN_ERR_IO, e + " (" + h->index_path + ")");
      GANN_HIP(gann::launch_step_round(h->ix, h->pq.dev, h->dtype, q_dev, nq, h->luts.as<float>(), topk,
                                       L, h->lists.as<uint64_t>(), h->state.p, nns, dists, active,
                                       (const uint8_t*)slots_dev, s));
      continue;
    }
    std::atomic<int> failed{0};
    team.run([&](int t) {
      try {
        for (int32_t j = t; j < nq; j += nthreads) {
          const int32_t u = req[(size_t)j];
          if (u >= 0)
            src.read_record(u, Ly.nodes_per_page, Ly.node_len,
                            (uint8_t*)h->slots.p + (size_t)j * gann::kSectorBytes);
        }
      } catch (...) {
        failed = 1;
      }
    });
    if (failed) raise(GANN_ERR_IO, "page read failed for " + h->index_path);
    GANN_HIP(gann::launch_step_round(h->ix, h->pq.dev, h->dtype, q_dev, nq, h->luts.as<float>(), topk,
                                     L, h->lists.as<uint64_t>(), h->state.p, nns, dists, active,
                                     (const uint8_t*)slots_dev, s));
  }
  GANN_HIP(gann::launch_step_finish(nq, topk, h->state.p, nns, dists, found, nexp, nadc, s));
}

// Device scratch of one search: counters (0: entry fallback count, 1:
// step-wise active count, 2: query queue) and q - centroid of every query.
// The handle's own buffers grow on demand; the fixed scratch of the
// allocation-free entry point is never grown (its caller checks the size)
// and serves the fused modes only.
struct SearchScratch {
  gann_handle* h;
  int32_t* fixed_counters = nullptr;
  float* fixed_qs = nullptr;
  bool fixed() const { return fixed_counters != nullptr; }
  int32_t* counters() {
    if (fixed()) return fixed_counters;
    h->counters.ensure(64);
    return h->counters.as<int32_t>();
  }
  float* qs(int64_t nfloats) {
    if (fixed()) return fixed_qs;
    h->qs.ensure((size_t)nfloats * 4);
    return h->qs.as<float>();
  }
  const int32_t* query_order = nullptr;  // set by order_queries for this call
};

// The order in which the fused kernels take the queries of this call:
// farthest from its entry point first (query_order_kernel in
// gann_kernels.hip).  Not in the allocation-free calls, which keep the
// queue's order; GANN_QUERY_ORDER=0 keeps it too.  Results are the same
// either way.
void order_queries(gann_handle* h, SearchScratch& sc, const float* q_dev, int32_t nq, const int32_t* entries,
                   hipStream_t s) {
  sc.query_order = nullptr;
  const char* e = std::getenv("GANN_QUERY_ORDER");
  if (sc.fixed() || (e && std::string(e) == "0")) return;
  h->entry_dist.ensure((size_t)nq * 4);
  h->order.ensure((size_t)nq * 4);
  GANN_HIP(gann::launch_query_order(h->ix, h->dtype, q_dev, nq, entries, h->entry_dist.as<float>(),
                                    h->order.as<int32_t>(), s));
  sc.query_order = h->order.as<int32_t>();
}

void run_search(gann_handle* h, SearchScratch& sc, const float* q_dev, int32_t nq, int32_t topk,
                int32_t L, int32_t mode, const int32_t* entries, int32_t* nns, float* dists,
                int32_t* found, int32_t* nexp, int32_t* nadc, hipStream_t s, int32_t beam = 1) {
  const gann::DiskLayout& Ly = h->layout;
  // Shared-codebook kernels: one workgroup per CU holding the pivot table and
  // as many lists as fit; below kMinLdsWaves lists, the pivots are read
  // through the caches and the LDS holds lists only.
  constexpr int kMinLdsWaves = 8;
  const int M = h->pq.dev.M, cw = h->pq.dev.chunk_w, D = (int)Ly.dim;
  const int w_lds = gann::search_cb_waves(D, M, cw, L, topk, h->lds_limit, false, 0);
  const int w_gp = gann::search_cb_waves(D, M, cw, L, topk, h->lds_limit, true, 0);
  if (beam > 1) {
    // beam search: shared-codebook kernel only
    if (mode != GANN_MODE_FUSED && mode != GANN_MODE_FUSED_GP)
      raise(GANN_ERR_UNSUPPORTED, "beam_width > 1 runs only in GANN_MODE_FUSED or GANN_MODE_FUSED_GP");
    const bool gp = mode == GANN_MODE_FUSED_GP || (w_lds < kMinLdsWaves && w_gp > w_lds);
    const int waves = gp ? w_gp : w_lds;
    if (waves < 1) raise(GANN_ERR_UNSUPPORTED, "beam_width > 1 needs one list in LDS");
    int32_t* ctr = sc.counters();
    float* qs = sc.qs((int64_t)nq * Ly.dim);
    const int blocks = std::max(1, std::min(h->num_cus, (nq + waves - 1) / waves));
    order_queries(h, sc, q_dev, nq, entries, s);
    GANN_HIP(gann::launch_search_beam(h->ix, h->pq.dev, h->dtype, q_dev, nq, entries, topk, L, beam,
                                      nns, dists, found, nexp, nadc, ctr + 2, sc.query_order, qs, waves,
                                      blocks, gp, s));
    return;
  }
  if (mode == GANN_MODE_FUSED || mode == GANN_MODE_FUSED_GP) {
    // Below kSplitWaves lists beside the whole table, keep all but its last
    // group of 8 chunks in LDS, or else its first half, when that leaves room
    // for kSplitWaves lists (measured on the 10M uint8 index: the half table
    // with 11 lists beats the cache-read table with 16 at L=1024); the groups
    // not in LDS are read through the caches.
    constexpr int kSplitWaves = 11;
    const int chunk_w = h->pq.dev.chunk_w;
    // split forms: one 64-neighbour block per expansion only (R <= 64)
    const int groups = Ly.max_m <= 64 ? gann::search_cb_split_groups(h->pq.dev.M, chunk_w) : 0;
    bool gp = mode == GANN_MODE_FUSED_GP || (w_lds < kMinLdsWaves && w_gp > w_lds);
    int g = 0;
    // Failing that, the half table while it keeps kHalfWaves lists: at dim
    // 128 it beats the wide form below down to 7 lists (10M index: L=1152,
    // 9 lists, 25.0 against 29.0 ms; L=1408, 7 lists, 32.2 against 35.5 ms;
    // L=1536 even) and loses at 6 (L=1664, 44.8 against 41.0 ms).
    constexpr int kHalfWaves = 7;
    if (mode == GANN_MODE_FUSED && w_lds < kSplitWaves && groups > 1) {
      for (int c : {groups - 1, groups / 2})
        if (gann::search_cb_waves(D, M, cw, L, topk, h->lds_limit, true, c) >= kSplitWaves) {
          g = c;
          gp = true;
          break;
        }
      if (g == 0 && gann::search_cb_waves(D, M, cw, L, topk, h->lds_limit, true, groups / 2) >= kHalfWaves) {
        g = groups / 2;
        gp = true;
      }
    }
    // Where the table would be read through the caches (no split keeps
    // enough lists), the wide form: 8-wave workgroups with every pivot row
    // of a lookup in flight and the first chunks in the LDS the lists leave.
    // Measured on uint8 dim-128 indexes it beats the cache-read form with
    // more lists at every L from 1024 to 2048 (10M index, 9-16 lists against
    // 8: 2-7% faster) and keeps its 8 lists above (7 at L=2576).
    const bool wide_ok = gann::search_cb_wide_ok(M, cw, D);
    if (mode == GANN_MODE_FUSED && gp && g == 0 && wide_ok) g = gann::kCbGpWide;
    // tuning override: "split" (all groups but one in LDS), "half",
    // "cache" (none in LDS) or "wide" (none in LDS, wide lookup) forces that
    // form
    if (const char* e = std::getenv("GANN_PIVOT_FORM")) {
      if (!std::strcmp(e, "split") && groups > 1) {
        g = groups - 1;
        gp = true;
      } else if (!std::strcmp(e, "half") && groups > 1) {
        g = groups / 2;
        gp = true;
      } else if (!std::strcmp(e, "cache")) {
        g = 0;
        gp = true;
      } else if (!std::strcmp(e, "wide") && wide_ok) {
        g = gann::kCbGpWide;
        gp = true;
      }
    }
    int waves = gp ? gann::search_cb_waves(D, M, cw, L, topk, h->lds_limit, true, g) : w_lds;
    // tuning override: GANN_CB_WAVES=n caps the lists (waves) per CU
    if (const char* e = std::getenv("GANN_CB_WAVES")) {
      const int cap = std::atoi(e);
      if (cap >= 1) waves = std::min(waves, cap);
    }
    // the wide form keeps its first chunks in the LDS the lists leave, up to
    // gann::kCbMaxWideLds of them (GANN_WIDE_LDS=n caps that, 0: none)
    if (gp && g == gann::kCbGpWide && waves >= 1) {
      int nl = gann::search_cb_wide_lds_chunks(cw, L, topk, h->lds_limit, waves, (int)h->ix.R);
      if (const char* e = std::getenv("GANN_WIDE_LDS")) nl = std::min(nl, std::max(0, std::atoi(e)));
      g = gann::kCbGpWide - nl;
    }
    if (waves >= 1 && (gp || waves >= 2)) {
      int32_t* ctr = sc.counters();
      float* qs = sc.qs((int64_t)nq * Ly.dim);
      const int blocks = std::max(1, std::min(h->num_cus, (nq + waves - 1) / waves));
      order_queries(h, sc, q_dev, nq, entries, s);
      GANN_HIP(gann::launch_search_cb(h->ix, h->pq.dev, h->dtype, q_dev, nq, entries, topk, L, nns,
                                      dists, found, nexp, nadc, ctr + 2, sc.query_order, qs, waves,
                                      blocks, gp, gp ? g : 0, s));
      return;
    }
    if (mode == GANN_MODE_FUSED_GP)
      raise(GANN_ERR_UNSUPPORTED, "GANN_MODE_FUSED_GP: one list does not fit in LDS");
    mode = GANN_MODE_FUSED_LUT;
  }
  if (mode == GANN_MODE_FUSED_LUT) {
    check_lds(gann::search_smem_bytes(h->pq.dev.M, (int)Ly.dim, L, (int)Ly.max_m, topk), h->device,
              "fused search");
    GANN_HIP(gann::launch_search(h->ix, h->pq.dev, h->dtype, q_dev, nq, entries, topk, L, nns,
                                 dists, found, nexp, nadc, s));
    return;
  }
  if (sc.fixed())
    raise(GANN_ERR_UNSUPPORTED, "the step-wise modes keep per-query LUTs and lists in scratch "
                                "allocated by the handle: use gann_search_device_ex for them");
  if (mode == GANN_MODE_STEPWISE_PAGED || mode == GANN_MODE_STEPWISE_URING) {
    run_stepwise_paged(h, q_dev, nq, topk, L, entries, nns, dists, found, nexp, nadc, s,
                       mode == GANN_MODE_STEPWISE_URING);
    return;
  }
  if (mode != GANN_MODE_STEPWISE) raise(GANN_ERR_INVALID, "unknown mode");
  // step-wise: LUTs in HBM, one launch per expansion round, host polls the
  // active count (the request[] round trip of src/hyd_task_runner.cu:126-178)
  h->luts.ensure((size_t)nq * h->pq.dev.M * gann::kNumPivots * 4);
  h->lists.ensure((size_t)nq * L * 8);
  h->state.ensure((size_t)nq * gann::step_state_bytes());
  h->counters.ensure(64);
  GANN_HIP(gann::launch_step_init(h->pq.dev, q_dev, nq, entries, h->luts.as<float>(), h->state.p, s));
  int32_t* active = h->counters.as<int32_t>() + 1;
  GANN_HIP(gann::launch_fill_i32(active, 1, nq, s));
  int32_t* host_active = (int32_t*)h->counter_host.p;
  const int64_t max_rounds = Ly.num_pts + 2;
  const int rounds_per_poll = 8;
  for (int64_t r = 0; r < max_rounds; r += rounds_per_poll) {
    for (int k = 0; k < rounds_per_poll; ++k)
      GANN_HIP(gann::launch_step_round(h->ix, h->pq.dev, h->dtype, q_dev, nq, h->luts.as<float>(),
                                       topk, L, h->lists.as<uint64_t>(), h->state.p, nns, dists,
                                       active, nullptr, s));
    GANN_HIP(hipMemcpyAsync(host_active, active, 4, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipStreamSynchronize(s));
    if (*host_active <= 0) break;
  }
  GANN_HIP(gann::launch_step_finish(nq, topk, h->state.p, nns, dists, found, nexp, nadc, s));
}

}  // namespace

extern "C" {

const char* gann_last_error(void) { return g_err.c_str(); }
const char* gann_version(void) { return "gustann-mi355x 0.1 (gfx950)"; }

int gann_open(const gann_config* cfg, gann_handle** out) {
  if (!out) {
    g_err = "out is NULL";
    return GANN_ERR_INVALID;
  }
  *out = nullptr;
  gann_handle* h = nullptr;
  int rc = guarded([&] {
    h = new gann_handle();
    open_handle(cfg, h);
  });
  if (rc != GANN_OK) {
    delete h;
    return rc;
  }
  *out = h;
  return GANN_OK;
}

int gann_close(gann_handle* h) {
  if (!h) return GANN_OK;
  return guarded([&] {
    GANN_HIP(hipSetDevice(h->device));
    delete h;
  });
}

int gann_get_info(const gann_handle* h, gann_index_info* info) {
  if (!h || !info) {
    g_err = "NULL argument";
    return GANN_ERR_INVALID;
  }
  const gann::DiskLayout& L = h->layout;
  info->num_pts = L.num_pts;
  info->dim = L.dim;
  info->medoid = L.medoid;
  info->max_m = L.max_m;
  info->node_len = L.node_len;
  info->nodes_per_page = L.nodes_per_page;
  info->num_pages = L.num_pages;
  info->dtype = h->dtype;
  info->num_chunks = h->pq.dev.M;
  info->nav_num_node = h->has_nav ? h->nav_host_meta.num_node : 0;
  info->nav_max_m = h->has_nav ? h->nav_host_meta.max_m : 0;
  info->nav_start = h->has_nav ? h->nav_host_meta.start : 0;
  return GANN_OK;
}

int gann_search_ex(gann_handle* h, const float* q, int32_t nq, int32_t topk, int32_t L,
                   int32_t beam_width, int32_t mode, int32_t* nns, float* dists,
                   int32_t* found_cnt, int32_t* n_exp, gann_stats* st) {
  return guarded([&] {
    if (!h) raise(GANN_ERR_INVALID, "handle is NULL");
    validate_search(h, nq, topk, L, beam_width);
    if (st) *st = gann_stats{};
    if (nq == 0) return;
    if (!q || !nns || !dists || !found_cnt) raise(GANN_ERR_INVALID, "NULL buffer");
    GANN_HIP(hipSetDevice(h->device));
    const int64_t D = h->layout.dim;
    hipStream_t s = h->stream;
    h->q.ensure((size_t)nq * D * 4);
    h->entries.ensure((size_t)nq * 4);
    h->nns.ensure((size_t)nq * topk * 4);
    h->dists.ensure((size_t)nq * topk * 4);
    h->found.ensure((size_t)nq * 4);
    h->nexp.ensure((size_t)nq * 4);
    h->nadc.ensure((size_t)nq * 4);
    h->counters.ensure(64);
    // query upload is outside the timed scope (src/pure_mem.cu:78-79)
    GANN_HIP(hipMemcpyAsync(h->q.p, q, (size_t)nq * D * 4, hipMemcpyHostToDevice, s));
    GANN_HIP(hipStreamSynchronize(s));
    const double t0 = now_s();
    run_entries(h, h->q.as<float>(), nq, h->entries.as<int32_t>(), nullptr, h->counters.as<int32_t>(), s);
    GANN_HIP(hipStreamSynchronize(s));
    const double t1 = now_s();
    SearchScratch sc{h};
    run_search(h, sc, h->q.as<float>(), nq, topk, L, mode, h->entries.as<int32_t>(),
               h->nns.as<int32_t>(), h->dists.as<float>(), h->found.as<int32_t>(),
               h->nexp.as<int32_t>(), h->nadc.as<int32_t>(), s, beam_width);
    GANN_HIP(hipStreamSynchronize(s));
    const double t2 = now_s();
    GANN_HIP(hipMemcpyAsync(nns, h->nns.p, (size_t)nq * topk * 4, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipMemcpyAsync(dists, h->dists.p, (size_t)nq * topk * 4, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipMemcpyAsync(found_cnt, h->found.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s));
    std::vector<int32_t> ne((size_t)nq), na((size_t)nq);
    int32_t fb = 0;
    GANN_HIP(hipMemcpyAsync(ne.data(), h->nexp.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipMemcpyAsync(na.data(), h->nadc.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipMemcpyAsync(&fb, h->counters.p, 4, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipStreamSynchronize(s));
    if (n_exp) std::memcpy(n_exp, ne.data(), (size_t)nq * 4);
    if (st) {
      st->run_time_s = t2 - t0;
      st->entry_time_s = t1 - t0;
      int64_t e = 0, a = 0;
      for (int32_t i = 0; i < nq; ++i) {
        e += ne[(size_t)i];
        a += na[(size_t)i];
      }
      st->n_expansions = e;
      st->n_adc = a;
      const double rec = (double)h->layout.data_len + 4.0;
      st->alg_bytes = (double)e * rec + (double)a * (4.0 + h->pq.dev.M) +
                      (double)nq * (4.0 * (double)D + 8.0 * topk);
      st->n_nav_fallback = fb;
    }
  });
}

int gann_search(gann_handle* h, const float* q, int32_t nq, int32_t topk, int32_t L,
                int32_t beam_width, int32_t* nns, float* dists, int32_t* found_cnt,
                gann_stats* st) {
  return gann_search_ex(h, q, nq, topk, L, beam_width, GANN_MODE_FUSED, nns, dists, found_cnt,
                        nullptr, st);
}

int gann_search_device_ex(gann_handle* h, const float* q_dev, int32_t nq, int32_t topk, int32_t L,
                          int32_t beam_width, int32_t mode, int32_t* entries_dev, int32_t* nns_dev,
                          float* dists_dev, int32_t* found_dev, int32_t* n_exp_dev,
                          int32_t* n_adc_dev, void* stream) {
  return guarded([&] {
    if (!h) raise(GANN_ERR_INVALID, "handle is NULL");
    validate_search(h, nq, topk, L, beam_width);
    if (nq == 0) return;
    if (!q_dev || !entries_dev || !nns_dev || !dists_dev || !found_dev)
      raise(GANN_ERR_INVALID, "NULL buffer");
    GANN_HIP(hipSetDevice(h->device));
    hipStream_t s = (hipStream_t)stream;
    SearchScratch sc{h};
    if (!(mode & GANN_SEARCH_ENTRIES_GIVEN))
      run_entries(h, q_dev, nq, entries_dev, nullptr, sc.counters(), s);
    run_search(h, sc, q_dev, nq, topk, L, mode & ~GANN_SEARCH_ENTRIES_GIVEN, entries_dev, nns_dev,
               dists_dev, found_dev, n_exp_dev, n_adc_dev, s, beam_width);
  });
}

int gann_search_device_noalloc(gann_handle* h, const float* q_dev, int32_t nq, int32_t topk, int32_t L,
                               int32_t beam_width, int32_t mode, int32_t* entries_dev, int32_t* nns_dev,
                               float* dists_dev, int32_t* found_dev, int32_t* n_exp_dev,
                               int32_t* n_adc_dev, void* stream) {
  return guarded([&] {
    if (!h) raise(GANN_ERR_INVALID, "handle is NULL");
    validate_search(h, nq, topk, L, beam_width);
    const bool given = (mode & GANN_SEARCH_ENTRIES_GIVEN) != 0;
    mode &= ~GANN_SEARCH_ENTRIES_GIVEN;
    if (mode != GANN_MODE_FUSED && mode != GANN_MODE_FUSED_GP && mode != GANN_MODE_FUSED_LUT)
      raise(GANN_ERR_UNSUPPORTED, "gann_search_device_noalloc runs the fused modes only "
                                  "(GANN_MODE_FUSED, GANN_MODE_FUSED_GP, GANN_MODE_FUSED_LUT)");
    const int64_t qs_bytes = (int64_t)nq * h->layout.dim * 4;
    const int64_t cap = (int64_t)(gann::kNoAllocScratchBytes - gann::kNoAllocCounterBytes);
    if (qs_bytes > cap)
      raise(GANN_ERR_INVALID, "gann_search_device_noalloc: nq * dim * 4 = " + std::to_string(qs_bytes) +
                                  " bytes exceeds its fixed scratch of " + std::to_string(cap) +
                                  " bytes (at most " + std::to_string(cap / (h->layout.dim * 4)) +
                                  " queries of this index per call)");
    if (nq == 0) return;
    if (!q_dev || !entries_dev || !nns_dev || !dists_dev || !found_dev)
      raise(GANN_ERR_INVALID, "NULL buffer");
    if (!h->noalloc_scratch) raise(GANN_ERR_HIP, "fixed scratch was not resolved for this device");
    GANN_HIP(hipSetDevice(h->device));
    hipStream_t s = (hipStream_t)stream;
    uint8_t* base = (uint8_t*)h->noalloc_scratch;
    SearchScratch sc{h, (int32_t*)base, (float*)(base + gann::kNoAllocCounterBytes)};
    if (!given) run_entries(h, q_dev, nq, entries_dev, nullptr, sc.counters(), s);
    run_search(h, sc, q_dev, nq, topk, L, mode, entries_dev, nns_dev, dists_dev, found_dev, n_exp_dev,
               n_adc_dev, s, beam_width);
  });
}

int gann_search_device(gann_handle* h, const float* q_dev, int32_t nq, int32_t topk, int32_t L,
                       int32_t* entries_dev, int32_t* nns_dev, float* dists_dev,
                       int32_t* found_dev, int32_t* n_exp_dev, int32_t* n_adc_dev, void* stream) {
  return gann_search_device_ex(h, q_dev, nq, topk, L, 1, GANN_MODE_FUSED, entries_dev, nns_dev,
                               dists_dev, found_dev, n_exp_dev, n_adc_dev, stream);
}

int gann_nav_entry(gann_handle* h, const float* q, int32_t nq, int32_t* entries_out,
                   int32_t* local_out) {
  return guarded([&] {
    if (!h) raise(GANN_ERR_INVALID, "handle is NULL");
    if (nq < 0) raise(GANN_ERR_INVALID, "nq must be >= 0");
    if (nq == 0) return;
    if (!q || !entries_out) raise(GANN_ERR_INVALID, "NULL buffer");
    GANN_HIP(hipSetDevice(h->device));
    hipStream_t s = h->stream;
    const int64_t D = h->layout.dim;
    h->q.ensure((size_t)nq * D * 4);
    h->entries.ensure((size_t)nq * 4);
    h->local.ensure((size_t)nq * 4);
    h->counters.ensure(64);
    GANN_HIP(hipMemcpyAsync(h->q.p, q, (size_t)nq * D * 4, hipMemcpyHostToDevice, s));
    run_entries(h, h->q.as<float>(), nq, h->entries.as<int32_t>(), h->local.as<int32_t>(),
                h->counters.as<int32_t>(), s);
    GANN_HIP(hipMemcpyAsync(entries_out, h->entries.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s));
    if (local_out)
      GANN_HIP(hipMemcpyAsync(local_out, h->local.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipStreamSynchronize(s));
  });
}

// ---------------------------------------------------------------- PQ entry points

int gann_pq_open(const char* pq_prefix, int32_t device_id, gann_pq** out) {
  if (!out) {
    g_err = "out is NULL";
    return GANN_ERR_INVALID;
  }
  *out = nullptr;
  gann_pq* p = nullptr;
  int rc = guarded([&] {
    if (!pq_prefix || !*pq_prefix) raise(GANN_ERR_INVALID, "pq_prefix is empty");
    int ndev = 0;
    GANN_HIP(hipGetDeviceCount(&ndev));
    if (device_id < 0 || device_id >= ndev) raise(GANN_ERR_INVALID, "device_id out of range");
    GANN_HIP(hipSetDevice(device_id));
    p = new gann_pq();
    p->device = device_id;
    GANN_HIP(hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking));
    gann::PQHost pqh;
    std::string err, pp(pq_prefix);
    if (!gann::read_pq(pp + "_pivots.bin", pp + "_compressed.bin", &pqh, true, &err))
      raise(err.rfind("cannot open", 0) == 0 ? GANN_ERR_IO : GANN_ERR_FORMAT, err);
    check_chunks(pqh.chunk_offsets.data(), pqh.dim, pqh.num_chunks);
    p->upload_static(pqh.pivots.data(), pqh.centroid.data(), pqh.chunk_offsets.data(), pqh.dim,
                     pqh.num_chunks);
    upload(p->codes, pqh.codes.data(), pqh.codes.size());
    p->dev.codes = p->codes.as<uint8_t>();
    p->dev.num_pts = pqh.num_pts;
  });
  if (rc != GANN_OK) {
    delete p;
    return rc;
  }
  *out = p;
  return GANN_OK;
}

int gann_pq_create(const float* pivots, const float* centroid, const int32_t* chunk_offsets,
                   int32_t dim, int32_t num_chunks, const uint8_t* codes, int64_t num_pts,
                   int32_t codes_on_device, int32_t device_id, gann_pq** out) {
  if (!out) {
    g_err = "out is NULL";
    return GANN_ERR_INVALID;
  }
  *out = nullptr;
  gann_pq* p = nullptr;
  int rc = guarded([&] {
    if (!pivots || !centroid || !chunk_offsets || (!codes && num_pts > 0))
      raise(GANN_ERR_INVALID, "NULL array");
    if (num_pts < 0 || num_pts >= (int64_t(1) << 31)) raise(GANN_ERR_INVALID, "num_pts out of range");
    check_chunks(chunk_offsets, dim, num_chunks);
    int ndev = 0;
    GANN_HIP(hipGetDeviceCount(&ndev));
    if (device_id < 0 || device_id >= ndev) raise(GANN_ERR_INVALID, "device_id out of range");
    GANN_HIP(hipSetDevice(device_id));
    p = new gann_pq();
    p->device = device_id;
    GANN_HIP(hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking));
    p->upload_static(pivots, centroid, chunk_offsets, dim, num_chunks);
    if (codes_on_device) {
      p->dev.codes = codes;
      p->codes_borrowed = true;
    } else {
      upload(p->codes, codes, (size_t)num_pts * num_chunks);
      p->dev.codes = p->codes.as<uint8_t>();
    }
    p->dev.num_pts = num_pts;
  });
  if (rc != GANN_OK) {
    delete p;
    return rc;
  }
  *out = p;
  return GANN_OK;
}

int gann_pq_close(gann_pq* pq) {
  if (!pq) return GANN_OK;
  return guarded([&] {
    GANN_HIP(hipSetDevice(pq->device));
    delete pq;
  });
}

int gann_handle_pq(gann_handle* h, gann_pq** out) {
  if (!h || !out) {
    g_err = "NULL argument";
    return GANN_ERR_INVALID;
  }
  *out = &h->pq;
  return GANN_OK;
}

int gann_pq_lut_build(gann_pq* pq, const float* q, int32_t nq, float* lut_out) {
  return guarded([&] {
    if (!pq) raise(GANN_ERR_INVALID, "pq is NULL");
    if (nq < 0) raise(GANN_ERR_INVALID, "nq must be >= 0");
    if (nq == 0) return;
    if (!q || !lut_out) raise(GANN_ERR_INVALID, "NULL buffer");
    GANN_HIP(hipSetDevice(pq->device));
    hipStream_t s = pq->stream;
    const size_t lut_bytes = (size_t)nq * pq->dev.M * gann::kNumPivots * 4;
    pq->q.ensure((size_t)nq * pq->dev.dim * 4);
    pq->out.ensure(lut_bytes);
    GANN_HIP(hipMemcpyAsync(pq->q.p, q, (size_t)nq * pq->dev.dim * 4, hipMemcpyHostToDevice, s));
    GANN_HIP(gann::launch_pq_lut(pq->dev, pq->q.as<float>(), nq, pq->out.as<float>(), s));
    GANN_HIP(hipMemcpyAsync(lut_out, pq->out.p, lut_bytes, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipStreamSynchronize(s));
  });
}

int gann_pq_adc_scan(gann_pq* pq, const float* q, int32_t nq, const int32_t* ids,
                     int32_t ids_per_q, float* out) {
  return guarded([&] {
    if (!pq) raise(GANN_ERR_INVALID, "pq is NULL");
    if (nq < 0 || ids_per_q < 0) raise(GANN_ERR_INVALID, "nq and ids_per_q must be >= 0");
    if (nq == 0 || ids_per_q == 0) return;
    if (!q || !ids || !out) raise(GANN_ERR_INVALID, "NULL buffer");
    const int64_t n = (int64_t)nq * ids_per_q;
    for (int64_t i = 0; i < n; ++i)
      if (ids[i] < 0 || ids[i] >= pq->dev.num_pts)
        raise(GANN_ERR_INVALID, "candidate id out of range at position " + std::to_string(i));
    GANN_HIP(hipSetDevice(pq->device));
    check_lds(gann::adc_smem_bytes(pq->dev.M, pq->dev.dim), pq->device, "ADC scan");
    hipStream_t s = pq->stream;
    pq->q.ensure((size_t)nq * pq->dev.dim * 4);
    pq->ids.ensure((size_t)n * 4);
    pq->out.ensure((size_t)n * 4);
    GANN_HIP(hipMemcpyAsync(pq->q.p, q, (size_t)nq * pq->dev.dim * 4, hipMemcpyHostToDevice, s));
    GANN_HIP(hipMemcpyAsync(pq->ids.p, ids, (size_t)n * 4, hipMemcpyHostToDevice, s));
    GANN_HIP(gann::launch_pq_adc_scan(pq->dev, pq->q.as<float>(), nq, pq->ids.as<int32_t>(), ids_per_q,
                                      pq->out.as<float>(), s));
    GANN_HIP(hipMemcpyAsync(out, pq->out.p, (size_t)n * 4, hipMemcpyDeviceToHost, s));
    GANN_HIP(hipStreamSynchronize(s));
  });
}

int gann_pq_adc_scan_device(gann_pq* pq, const float* q_dev, int32_t nq, const int32_t* ids_dev,
                            int32_t ids_per_q, float* out_dev, void* stream) {
  return guarded([&] {
    if (!pq) raise(GANN_ERR_INVALID, "pq is NULL");
    if (nq < 0 || ids_per_q < 0) raise(GANN_ERR_INVALID, "nq and ids_per_q must be >= 0");
    if (nq == 0 || ids_per_q == 0) return;
    if (!q_dev || !ids_dev || !out_dev) raise(GANN_ERR_INVALID, "NULL buffer");
    GANN_HIP(hipSetDevice(pq->device));
    check_lds(gann::adc_smem_bytes(pq->dev.M, pq->dev.dim), pq->device, "ADC scan");
    hipStream_t s = (hipStream_t)stream;
    GANN_HIP(gann::launch_pq_adc_scan(pq->dev, q_dev, nq, ids_dev, ids_per_q, out_dev, s));
  });
}


namespace {

// Slices of a base chunk for the exact k-NN: each (query block, slice) is one
// wavefront.  The count minimizes ceil(qblocks s / resident) / s, the rounds
// of resident wavefronts times the points per slice (a last round far from
// full idles the GPU), over at most 3 rounds (every slice adds candidate
// insertions), with at least 1024 points per slice; the smallest count on a
// tie.
int64_t knn_slices(int64_t qblocks, int64_t resident, int64_t chunk) {
  const int64_t smax = std::max<int64_t>(1, std::min<int64_t>((chunk + 1023) / 1024, 3 * resident / qblocks));
  int64_t best = 1, best_r = (qblocks + resident - 1) / resident;
  for (int64_t s = 2; s <= smax; ++s) {
    const int64_t r = (qblocks * s + resident - 1) / resident;
    if (r * best < best_r * s) best = s, best_r = r;
  }
  return best;
}

}  // namespace

int gann_knn_exact(const void* base, int64_t n, int32_t dim, int32_t dtype, const float* queries,
                   int32_t nq, int32_t k, int32_t device_id, int32_t* ids, float* dists) {
  return guarded([&] {
    if (dtype != GANN_UINT8 && dtype != GANN_FLOAT) raise(GANN_ERR_INVALID, "unknown data type");
    if (n < 1 || nq < 0) raise(GANN_ERR_INVALID, "need n >= 1 and nq >= 0");
    if (dim < 1 || dim > 256) raise(GANN_ERR_UNSUPPORTED, "dim must be in [1, 256]");
    if (k < 1 || k > 128) raise(GANN_ERR_UNSUPPORTED, "k must be in [1, 128]");
    if (n > (int64_t)INT32_MAX) raise(GANN_ERR_UNSUPPORTED, "ids are int32: n must be < 2^31");
    if (nq == 0) return;
    if (!base || !queries || !ids || !dists) raise(GANN_ERR_INVALID, "NULL buffer");
    const bool u8 = dtype == GANN_UINT8;
    if (u8)
      for (int64_t i = 0; i < (int64_t)nq * dim; ++i) {
        const float v = queries[i];
        if (!(v >= 0.0f && v <= 255.0f) || v != std::floor(v))
          raise(GANN_ERR_INVALID, "uint8 queries must hold integers in [0, 255]");
      }
    GANN_HIP(hipSetDevice(device_id));
    int cus = 0;
    GANN_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device_id));
    const gann::KnnU8Form form = u8 ? gann::knn_u8_form(dim, k) : gann::KnnU8Form{0, 0, 0};
    if (u8 && form.blocks_per_cu < 1) raise(GANN_ERR_UNSUPPORTED, "exact k-NN kernel does not fit a CU");
    const int QB = u8 ? form.qb : gann::kKnnF32Queries;
    const int nqp = (nq + QB - 1) / QB * QB;
    const int dp = form.dp;
    const size_t elem = u8 ? 1 : 4;
    int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(n, ((int64_t)1 << 31) / (dim * (int64_t)elem)));
    if (const char* e = std::getenv("GANN_KNN_CHUNK"))  // smaller chunks: tests of the chunk merge
      chunk = std::max<int64_t>(1, std::min<int64_t>(chunk, std::atoll(e)));
    const int64_t qblocks = nqp / QB;
    const int64_t resident =
        (int64_t)cus * std::max(1, u8 ? form.blocks_per_cu : gann::knn_f32_blocks_per_cu(dim, k));
    int64_t slices = knn_slices(qblocks, resident, chunk);
    const int64_t slice_len = ((chunk + slices - 1) / slices + 31) / 32 * 32;
    slices = (chunk + slice_len - 1) / slice_len;
    // part_d/part_i hold [slices + 1][nq][k]: slot 0 keeps the best of the
    // chunks merged so far, a chunk's slices go to slots 1.. (0.. for the
    // first chunk) and are merged into slot 0 on the device
    DevBuf raw, xs, xn, qs, qn, qf, pd, pi;
    raw.ensure((size_t)chunk * dim * elem);
    pd.ensure((size_t)(slices + 1) * nq * k * 4);
    pi.ensure((size_t)(slices + 1) * nq * k * 4);
    if (u8) {
      std::vector<int8_t> hq((size_t)nqp * dp, 0);
      std::vector<int32_t> hn((size_t)nqp, 0);
      for (int32_t q = 0; q < nq; ++q) {
        int32_t sum = 0;
        for (int32_t d = 0; d < dim; ++d) {
          const int v = (int)queries[(size_t)q * dim + d] - 128;
          hq[(size_t)q * dp + d] = (int8_t)v;
          sum += v * v;
        }
        hn[(size_t)q] = sum;
      }
      xs.ensure((size_t)chunk * dp);
      xn.ensure((size_t)chunk * 4);
      qs.ensure(hq.size());
      qn.ensure(hn.size() * 4);
      GANN_HIP(hipMemcpy(qs.p, hq.data(), hq.size(), hipMemcpyHostToDevice));
      GANN_HIP(hipMemcpy(qn.p, hn.data(), hn.size() * 4, hipMemcpyHostToDevice));
    } else {
      qf.ensure((size_t)nq * dim * 4);
      GANN_HIP(hipMemcpy(qf.p, queries, (size_t)nq * dim * 4, hipMemcpyHostToDevice));
    }
    check_lds(gann::knn_smem_bytes(u8 ? 0 : 1, QB, u8 ? dp : dim, k), device_id, "exact k-NN");
    for (int64_t off = 0; off < n; off += chunk) {
      const int64_t cn = std::min(chunk, n - off);
      const int64_t cs = (cn + slice_len - 1) / slice_len;
      const int64_t s0 = off == 0 ? 0 : 1;
      float* sd = pd.as<float>() + (size_t)s0 * nq * k;
      int32_t* si = pi.as<int32_t>() + (size_t)s0 * nq * k;
      GANN_HIP(hipMemcpy(raw.p, (const uint8_t*)base + (size_t)off * dim * elem, (size_t)cn * dim * elem,
                         hipMemcpyHostToDevice));
      if (u8) {
        GANN_HIP(gann::launch_knn_prep_u8(raw.as<uint8_t>(), cn, dim, dp, xs.as<int8_t>(),
                                          xn.as<int32_t>(), 0));
        GANN_HIP(gann::launch_knn_u8(form, xs.as<int8_t>(), xn.as<int32_t>(), cn, qs.as<int8_t>(),
                                     qn.as<int32_t>(), nq, k, cs, slice_len, off, sd, si, 0));
      } else {
        GANN_HIP(gann::launch_knn_f32(raw.as<float>(), cn, dim, qf.as<float>(), nq, k, cs, slice_len,
                                      off, sd, si, 0));
      }
      GANN_HIP(gann::launch_knn_merge(pd.as<float>(), pi.as<int32_t>(), nq, k, s0 + cs, 0));
    }
    GANN_HIP(hipMemcpy(ids, pi.p, (size_t)nq * k * 4, hipMemcpyDeviceToHost));
    GANN_HIP(hipMemcpy(dists, pd.p, (size_t)nq * k * 4, hipMemcpyDeviceToHost));
  });
}


namespace {

// Device copy of [n][dim] uint8 rows padded to dp bytes, with squared norms.
void upload_build_rows(const uint8_t* data, int64_t n, int dim, int dp, DevBuf& x, DevBuf& xn) {
  x.ensure((size_t)n * dp);
  xn.ensure((size_t)n * 4);
  if (dp == dim) {
    GANN_HIP(hipMemcpy(x.p, data, (size_t)n * dp, hipMemcpyHostToDevice));
  } else {
    GANN_HIP(hipMemset(x.p, 0, (size_t)n * dp));
    GANN_HIP(hipMemcpy2D(x.p, (size_t)dp, data, (size_t)dim, (size_t)dim, (size_t)n, hipMemcpyHostToDevice));
  }
  GANN_HIP(gann::launch_build_norms(x.as<uint8_t>(), n, dp, xn.as<int32_t>(), 0));
}

int device_lds_limit(int device) {
  int lim = 0;
  GANN_HIP(hipDeviceGetAttribute(&lim, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
  return lim;
}

}  // namespace

int gann_build_vamana(const uint8_t* data, int64_t n, int32_t dim, int32_t R, int32_t L, float alpha,
                      uint64_t seed, int64_t max_batch, int32_t device_id, int32_t verbose,
                      uint32_t* out_nbr, uint32_t* out_deg, int64_t* out_medoid) {
  return guarded([&] {
    if (!data || !out_nbr || !out_deg || !out_medoid) raise(GANN_ERR_INVALID, "NULL buffer");
    if (n < 1 || n >= (int64_t)INT32_MAX) raise(GANN_ERR_INVALID, "need 1 <= n < 2^31 - 1");
    const int dp = gann::build_row_bytes(dim);
    if (dp == 0) raise(GANN_ERR_UNSUPPORTED, "dim must be in [1, 256]");
    if (R < 1 || R > 64) raise(GANN_ERR_UNSUPPORTED, "R must be in [1, 64]");
    if (L < 1 || L > 1024) raise(GANN_ERR_UNSUPPORTED, "L must be in [1, 1024]");
    if (!std::isfinite(alpha) || !(alpha >= 1.0f)) raise(GANN_ERR_INVALID, "alpha must be finite and >= 1");
    if (max_batch < 1) raise(GANN_ERR_INVALID, "max_batch must be >= 1");
    const int64_t mb = std::min<int64_t>({max_batch, n, (int64_t)(INT32_MAX / 64)});
    GANN_HIP(hipSetDevice(device_id));
    int cus = 0;
    GANN_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device_id));
    const int lds = device_lds_limit(device_id);
    if (gann::build_prune_waves(dp, (size_t)lds) < 1)
      raise(GANN_ERR_UNSUPPORTED, "graph build: prune workspace exceeds the LDS limit");
    check_lds(gann::build_search_smem_bytes(L, 4), device_id, "graph build search");
    const auto t0 = std::chrono::steady_clock::now();
    auto secs = [&] {
      return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    };
    DevBuf x, xn, nbr, deg, ord, sums, mean, best;
    upload_build_rows(data, n, dim, dp, x, xn);
    const int C = gann::build_capacity(R);  // lists grow to C before a prune (graph slack)
    nbr.ensure((size_t)n * C * 4);
    deg.ensure((size_t)n * 4);
    // medoid: the point closest to the mean
    sums.ensure((size_t)dp * 8);
    GANN_HIP(hipMemset(sums.p, 0, (size_t)dp * 8));
    GANN_HIP(gann::launch_build_col_sums(x.as<uint8_t>(), n, dp, sums.as<unsigned long long>(), 0));
    std::vector<unsigned long long> hs((size_t)dp);
    GANN_HIP(hipMemcpy(hs.data(), sums.p, (size_t)dp * 8, hipMemcpyDeviceToHost));
    std::vector<float> hm((size_t)dim);
    for (int j = 0; j < dim; ++j) hm[(size_t)j] = (float)((double)hs[(size_t)j] / (double)n);
    mean.ensure((size_t)dim * 4);
    GANN_HIP(hipMemcpy(mean.p, hm.data(), (size_t)dim * 4, hipMemcpyHostToDevice));
    best.ensure(8);
    GANN_HIP(hipMemset(best.p, 0xff, 8));
    GANN_HIP(gann::launch_build_medoid(x.as<uint8_t>(), n, dim, dp, mean.as<float>(),
                                       best.as<unsigned long long>(), 0));
    unsigned long long hb = 0;
    GANN_HIP(hipMemcpy(&hb, best.p, 8, hipMemcpyDeviceToHost));
    const uint32_t medoid = (uint32_t)(hb & 0xffffffffull);
    if ((int64_t)medoid >= n) raise(GANN_ERR_FORMAT, "graph build: medoid search failed");
    // random initial graph and the insertion order
    const int init_deg = (int)std::min<int64_t>(R / 2 > 0 ? R / 2 : 1, n - 1);
    gann::BuildDev g{x.as<uint8_t>(), xn.as<int32_t>(), nbr.as<uint32_t>(), deg.as<uint32_t>(), n, dp, R, C};
    GANN_HIP(gann::launch_build_random_graph(g, init_deg, seed, 0));
    {
      std::vector<uint32_t> order((size_t)n);
      std::iota(order.begin(), order.end(), 0u);
      std::mt19937_64 gen(seed ^ 0x5eedull);
      std::shuffle(order.begin(), order.end(), gen);
      ord.ensure((size_t)n * 4);
      GANN_HIP(hipMemcpy(ord.p, order.data(), (size_t)n * 4, hipMemcpyHostToDevice));
    }
    DevBuf pool_id, pool_d, pool_n, pa, pb, flags, seg, nseg, queue, temp;
    pool_id.ensure((size_t)mb * gann::kBuildPoolMax * 4);
    pool_d.ensure((size_t)mb * gann::kBuildPoolMax * 4);
    pool_n.ensure((size_t)mb * 4);
    pa.ensure((size_t)mb * R * 8);
    pb.ensure((size_t)mb * R * 8);
    flags.ensure((size_t)mb * R);
    seg.ensure((size_t)mb * R * 4);
    nseg.ensure(4);
    queue.ensure(4);
    size_t tb = 0;
    GANN_HIP(gann::build_segments_temp_bytes(mb * R, &tb));
    temp.ensure(tb);
    if (verbose)
      std::fprintf(stderr, "[gpu-vamana] n %lld dim %d R %d L %d alpha %.2f batch %lld: setup %.1f s\n",
                   (long long)n, dim, R, L, (double)alpha, (long long)mb, secs());
    double last = secs();
    for (int pass = 0; pass < 2; ++pass) {
      const float a = pass == 0 ? 1.0f : alpha;
      int64_t off = 0, bs = pass == 0 ? 1 : mb;
      while (off < n) {
        const int64_t b = std::min(bs, n - off);
        const uint32_t* pts = ord.as<uint32_t>() + off;
        GANN_HIP(hipMemsetAsync(queue.p, 0, 4, 0));
        GANN_HIP(gann::launch_build_search(g, pts, (int)b, medoid, L, pool_id.as<uint32_t>(), pool_d.as<float>(),
                                           pool_n.as<int32_t>(), queue.as<int32_t>(), cus, 0));
        GANN_HIP(hipMemsetAsync(queue.p, 0, 4, 0));
        GANN_HIP(gann::launch_build_prune_fwd(g, pts, (int)b, pool_id.as<uint32_t>(), pool_d.as<float>(),
                                              pool_n.as<int32_t>(), a, pa.as<unsigned long long>(),
                                              queue.as<int32_t>(), cus, (size_t)lds, 0));
        GANN_HIP(gann::launch_build_segments(temp.p, tb, pa.as<unsigned long long>(), pb.as<unsigned long long>(),
                                             b * R, flags.as<uint8_t>(), seg.as<int32_t>(), nseg.as<int32_t>(), 0));
        GANN_HIP(hipMemsetAsync(queue.p, 0, 4, 0));
        GANN_HIP(gann::launch_build_reverse(g, pb.as<unsigned long long>(), b * R, seg.as<int32_t>(),
                                            nseg.as<int32_t>(), a, queue.as<int32_t>(), cus, (size_t)lds, 0));
        GANN_HIP(hipStreamSynchronize(0));
        off += b;
        if (pass == 0) bs = std::min(bs * 2, mb);
        if (verbose && (secs() - last > 10.0 || off == n)) {
          last = secs();
          std::fprintf(stderr, "[gpu-vamana] alpha %.2f: %lld / %lld (%.1f s)\n", (double)a, (long long)off,
                       (long long)n, last);
        }
      }
    }
    // every list back to at most R
    GANN_HIP(hipMemsetAsync(queue.p, 0, 4, 0));
    GANN_HIP(gann::launch_build_final_prune(g, alpha, queue.as<int32_t>(), cus, (size_t)lds, 0));
    GANN_HIP(hipDeviceSynchronize());
    if (verbose) std::fprintf(stderr, "[gpu-vamana] final prune done (%.1f s)\n", secs());
    pool_id.release();
    pool_d.release();
    pa.release();
    pb.release();
    temp.release();
    DevBuf packed;
    packed.ensure((size_t)n * R * 4);
    GANN_HIP(gann::launch_build_compact(g, packed.as<uint32_t>(), 0));
    GANN_HIP(hipMemcpy(out_nbr, packed.p, (size_t)n * R * 4, hipMemcpyDeviceToHost));
    GANN_HIP(hipMemcpy(out_deg, deg.p, (size_t)n * 4, hipMemcpyDeviceToHost));
    *out_medoid = (int64_t)medoid;
  });
}

int gann_pq_encode(const void* data, int64_t n, int32_t dim, int32_t dtype, const float* pivots,
                   const float* centroid, const int32_t* chunk_offsets, int32_t M, int32_t device_id,
                   uint8_t* codes) {
  return guarded([&] {
    if (dtype != GANN_UINT8 && dtype != GANN_FLOAT) raise(GANN_ERR_INVALID, "unknown data type");
    if (n < 0 || dim < 1 || M < 1 || M > dim) raise(GANN_ERR_INVALID, "need n >= 0 and 1 <= M <= dim");
    if (n == 0) return;
    if (!data || !pivots || !centroid || !chunk_offsets || !codes) raise(GANN_ERR_INVALID, "NULL buffer");
    if (chunk_offsets[0] != 0 || chunk_offsets[M] != dim)
      raise(GANN_ERR_INVALID, "chunk offsets must tile [0, dim)");
    for (int32_t m = 0; m < M; ++m) {
      const int32_t w = chunk_offsets[m + 1] - chunk_offsets[m];
      if (w < 0) raise(GANN_ERR_INVALID, "chunk offsets must not decrease");
      if (w > gann::kPqEncodeMaxW) raise(GANN_ERR_UNSUPPORTED, "chunks of at most 16 dims");
    }
    GANN_HIP(hipSetDevice(device_id));
    const size_t elem = dtype == GANN_UINT8 ? 1 : 4;
    const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(n, ((int64_t)1 << 30) / ((int64_t)dim * elem)));
    DevBuf dx, dp, dc, doff, dcodes;
    dx.ensure((size_t)chunk * dim * elem);
    dcodes.ensure((size_t)chunk * M);
    upload(dp, pivots, (size_t)gann::kNumPivots * dim * 4);
    upload(dc, centroid, (size_t)dim * 4);
    upload(doff, chunk_offsets, (size_t)(M + 1) * 4);
    for (int64_t off = 0; off < n; off += chunk) {
      const int64_t cn = std::min(chunk, n - off);
      GANN_HIP(hipMemcpy(dx.p, (const uint8_t*)data + (size_t)off * dim * elem, (size_t)cn * dim * elem,
                         hipMemcpyHostToDevice));
      GANN_HIP(gann::launch_pq_encode(dx.p, dtype == GANN_UINT8 ? 0 : 1, cn, dim, dp.as<float>(), dc.as<float>(),
                                      doff.as<int32_t>(), M, dcodes.as<uint8_t>(), 0));
      GANN_HIP(hipMemcpy(codes + (size_t)off * M, dcodes.p, (size_t)cn * M, hipMemcpyDeviceToHost));
    }
  });
}

int gann_diag_robust_prune(const uint8_t* data, int64_t n, int32_t dim, int64_t p, const uint32_t* cand,
                           int32_t ncand, float alpha, int32_t R, int32_t device_id, uint32_t* out,
                           int32_t* nout) {
  return guarded([&] {
    if (!data || !out || !nout || (ncand > 0 && !cand)) raise(GANN_ERR_INVALID, "NULL buffer");
    if (n < 1 || n >= (int64_t)INT32_MAX) raise(GANN_ERR_INVALID, "need 1 <= n < 2^31 - 1");
    if (p < 0 || p >= n) raise(GANN_ERR_INVALID, "p outside [0, n)");
    const int dp = gann::build_row_bytes(dim);
    if (dp == 0) raise(GANN_ERR_UNSUPPORTED, "dim must be in [1, 256]");
    if (R < 1 || R > 64) raise(GANN_ERR_UNSUPPORTED, "R must be in [1, 64]");
    if (ncand < 0 || ncand > gann::kBuildCandMax) raise(GANN_ERR_UNSUPPORTED, "ncand must be in [0, " + std::to_string(gann::kBuildCandMax) + "]");
    if (std::isnan(alpha)) raise(GANN_ERR_INVALID, "alpha is NaN");
    for (int32_t i = 0; i < ncand; ++i)
      if ((int64_t)cand[i] >= n) raise(GANN_ERR_INVALID, "candidate id outside [0, n)");
    GANN_HIP(hipSetDevice(device_id));
    const int lds = device_lds_limit(device_id);
    DevBuf x, xn, nbr, deg, dc, dout, dn;
    upload_build_rows(data, n, dim, dp, x, xn);
    nbr.ensure((size_t)n * R * 4);
    deg.ensure((size_t)n * 4);
    dc.ensure((size_t)std::max(ncand, 1) * 4);
    dout.ensure((size_t)R * 4);
    dn.ensure(4);
    if (ncand > 0) GANN_HIP(hipMemcpy(dc.p, cand, (size_t)ncand * 4, hipMemcpyHostToDevice));
    gann::BuildDev g{x.as<uint8_t>(), xn.as<int32_t>(), nbr.as<uint32_t>(), deg.as<uint32_t>(), n, dp, R, R};
    GANN_HIP(gann::launch_build_prune_one(g, (uint32_t)p, dc.as<uint32_t>(), ncand, alpha, dout.as<uint32_t>(),
                                          dn.as<int32_t>(), (size_t)lds, 0));
    int32_t k = 0;
    GANN_HIP(hipMemcpy(&k, dn.p, 4, hipMemcpyDeviceToHost));
    if (k < 0 || k > R) raise(GANN_ERR_FORMAT, "prune returned a bad count");
    if (k > 0) GANN_HIP(hipMemcpy(out, dout.p, (size_t)k * 4, hipMemcpyDeviceToHost));
    *nout = k;
  });
}

int gann_diag_gather_rows(const uint8_t* rows_dev, int64_t num_rows, int32_t row_bytes,
                          const int32_t* ids_dev, int64_t n_ids, uint32_t* out_dev, void* stream) {
  return guarded([&] {
    if (row_bytes != 16 && row_bytes != 32 && row_bytes != 48 && row_bytes != 64)
      raise(GANN_ERR_UNSUPPORTED, "row_bytes must be 16, 32, 48 or 64");
    if (num_rows < 1 || n_ids < 0) raise(GANN_ERR_INVALID, "need num_rows >= 1 and n_ids >= 0");
    if (n_ids == 0) return;
    if (!rows_dev || !ids_dev || !out_dev) raise(GANN_ERR_INVALID, "NULL buffer");
    GANN_HIP(gann::launch_gather_rows(rows_dev, num_rows, row_bytes, ids_dev, n_ids, out_dev,
                                      (hipStream_t)stream));
  });
}

}  // extern "C"
