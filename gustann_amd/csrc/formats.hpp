// Byte-exact readers and writers for the DiskANN-family files that GustANN's
// in-memory search consumes.  Host-only C++17, header-only, shared by the HIP
// runtime library (libgustann_hip.so) and the index builder
// (libgustann_index.so).
//
// Formats (all little-endian):
//  * "bin": int32 npts, int32 ndims, then npts*ndims elements.
//    Reference reader: src/pq_search.cu:187-201, bin/utils.hpp:90-101.
//  * <prefix>_disk.index: sector 0 = bin header (u32 nr, u32 nc) followed by
//    u64 npts, ndims, medoid, max_node_len, nnodes_per_sector, num_frozen,
//    frozen_loc, reorder_exists (src/layout.cpp:27-54); sectors 1.. hold
//    node records packed nnodes_per_sector per 4096-byte sector, record =
//    T coords[ndims] | u32 deg | u32 nbrs[R] (src/impl/pure_mem.cuh:261-292).
//  * <pq>_pivots.bin: bin of u64 offsets[nr] (nr = 4, or 5 for the legacy
//    layout with a rearrangement table) at 0; at offsets[0] a bin 256 x D f32
//    pivots, at offsets[1] a bin D x 1 f32 centroid, at offsets[2] (offsets[3]
//    when nr == 5) a bin (M+1) x 1 i32 chunk offsets (src/pq_search.cu:56-121).
//  * <pq>_compressed.bin: bin N x M u8 (src/pq_search.cu:61).
//  * nav/nav_index: u64 file_size, u32 max_degree, u32 start, u64 num_frozen,
//    then per node u32 k, u32 nbrs[k]; nav/nav_index.data: bin n x D of T;
//    nav/map.txt: n decimal base ids (src/nav_graph.cu:41-100).
//  * bvecs / fvecs / ivecs: per row i32 d then d elements (bin/utils.hpp:23-88).
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace gann {

constexpr int64_t kSectorBytes = 4096;
constexpr int kNumPivots = 256;

struct DiskLayout {
  int64_t num_pts = 0;
  int64_t dim = 0;
  int64_t medoid = 0;
  int64_t node_len = 0;        // bytes per node record (max_node_len)
  int64_t nodes_per_page = 0;  // records per 4096-byte sector
  int64_t max_m = 0;           // R = (node_len - dim*elem)/4 - 1
  int64_t data_len = 0;        // dim * elem bytes (coords prefix of a record)
  int64_t num_pages = 0;       // ceil(num_pts / nodes_per_page)
  int64_t elem_size = 1;       // 1 = uint8, 4 = float
};

struct PQHost {
  int dim = 0;
  int num_chunks = 0;
  int64_t num_pts = 0;
  std::vector<float> pivots;          // [256][dim], row-major as stored
  std::vector<float> centroid;        // [dim]
  std::vector<int32_t> chunk_offsets; // [num_chunks + 1]
  std::vector<uint8_t> codes;         // [num_pts][num_chunks]
};

struct NavHost {
  int64_t num_node = 0;
  int dim = 0;
  int max_m = 0;
  int start = 0;
  std::vector<uint8_t> data;     // [num_node][dim] of T (raw bytes)
  std::vector<int32_t> graph;    // [num_node][max_m], padded with -1
  std::vector<int32_t> mapping;  // [num_node] base ids
};

// ---------------------------------------------------------------- helpers

class File {
 public:
  File(const std::string& path, const char* mode) : f_(std::fopen(path.c_str(), mode)) {}
  ~File() {
    if (f_) std::fclose(f_);
  }
  File(const File&) = delete;
  File& operator=(const File&) = delete;
  explicit operator bool() const { return f_ != nullptr; }
  FILE* get() const { return f_; }
  bool read(void* dst, size_t bytes) { return bytes == 0 || std::fread(dst, 1, bytes, f_) == bytes; }
  bool write(const void* src, size_t bytes) { return bytes == 0 || std::fwrite(src, 1, bytes, f_) == bytes; }
  bool seek(int64_t off) { return fseeko(f_, (off_t)off, SEEK_SET) == 0; }
  int64_t size() {
    off_t cur = ftello(f_);
    fseeko(f_, 0, SEEK_END);
    off_t end = ftello(f_);
    fseeko(f_, cur, SEEK_SET);
    return (int64_t)end;
  }

 private:
  FILE* f_;
};

inline bool fail(std::string* err, const std::string& msg) {
  if (err) *err = msg;
  return false;
}

// Reads a bin header + payload at `offset`. `elem` is sizeof(T).
inline bool read_bin_raw(const std::string& path, int64_t offset, size_t elem, int32_t* npts,
                         int32_t* ndim, std::vector<uint8_t>* payload, std::string* err) {
  File f(path, "rb");
  if (!f) return fail(err, "cannot open " + path);
  if (!f.seek(offset)) return fail(err, "seek failed in " + path);
  int32_t hdr[2];
  if (!f.read(hdr, sizeof(hdr))) return fail(err, "truncated bin header in " + path);
  if (hdr[0] < 0 || hdr[1] < 0) return fail(err, "negative bin dimensions in " + path);
  *npts = hdr[0];
  *ndim = hdr[1];
  size_t bytes = (size_t)hdr[0] * (size_t)hdr[1] * elem;
  payload->resize(bytes);
  if (!f.read(payload->data(), bytes)) return fail(err, "truncated bin payload in " + path);
  return true;
}

template <class T>
inline bool read_bin(const std::string& path, int64_t offset, int32_t* npts, int32_t* ndim,
                     std::vector<T>* out, std::string* err) {
  std::vector<uint8_t> raw;
  if (!read_bin_raw(path, offset, sizeof(T), npts, ndim, &raw, err)) return false;
  out->resize(raw.size() / sizeof(T));
  if (!raw.empty()) std::memcpy(out->data(), raw.data(), raw.size());
  return true;
}

// Writes a bin at the current position of `f`; returns bytes written.
inline int64_t write_bin_at(File& f, int64_t offset, int32_t npts, int32_t ndim, const void* data,
                            size_t elem) {
  if (!f.seek(offset)) return -1;
  int32_t hdr[2] = {npts, ndim};
  if (!f.write(hdr, sizeof(hdr))) return -1;
  size_t bytes = (size_t)npts * (size_t)ndim * elem;
  if (!f.write(data, bytes)) return -1;
  return (int64_t)(sizeof(hdr) + bytes);
}

inline bool write_bin(const std::string& path, int32_t npts, int32_t ndim, const void* data,
                      size_t elem, std::string* err) {
  File f(path, "wb");
  if (!f) return fail(err, "cannot create " + path);
  if (write_bin_at(f, 0, npts, ndim, data, elem) < 0) return fail(err, "write failed: " + path);
  return true;
}

// ---------------------------------------------------------------- disk index

// Parses sector 0 (src/layout.cpp:11-69).  elem_size = sizeof(T).
inline bool parse_disk_meta(const std::string& path, int64_t elem_size, DiskLayout* L,
                            std::string* err) {
  File f(path, "rb");
  if (!f) return fail(err, "cannot open index file " + path);
  uint32_t nr_nc[2];
  uint64_t v[8];
  if (!f.read(nr_nc, sizeof(nr_nc)) || !f.read(v, sizeof(v)))
    return fail(err, "truncated disk-index metadata in " + path);
  L->num_pts = (int64_t)v[0];
  L->dim = (int64_t)v[1];
  L->medoid = (int64_t)v[2];
  L->node_len = (int64_t)v[3];
  L->nodes_per_page = (int64_t)v[4];
  L->elem_size = elem_size;
  L->data_len = L->dim * elem_size;
  if (L->num_pts <= 0 || L->num_pts >= (int64_t(1) << 31))
    return fail(err, "disk index: num_pts out of range (bit 31 of an id is the visited flag)");
  if (L->dim <= 0 || L->node_len <= L->data_len + 4 || L->node_len > kSectorBytes)
    return fail(err, "disk index: inconsistent dim / max_node_len");
  if ((L->node_len - L->data_len) % 4 != 0)
    return fail(err, "disk index: node length not a multiple of 4 past the coordinates");
  L->max_m = (L->node_len - L->data_len) / 4 - 1;  // src/layout.cpp:46
  if (L->nodes_per_page <= 0 || L->nodes_per_page * L->node_len > kSectorBytes)
    return fail(err, "disk index: nodes_per_sector inconsistent with max_node_len");
  if (L->medoid < 0 || L->medoid >= L->num_pts) return fail(err, "disk index: medoid out of range");
  L->num_pages = (L->num_pts + L->nodes_per_page - 1) / L->nodes_per_page;  // src/layout.cpp:60
  int64_t need = (L->num_pages + 1) * kSectorBytes;
  if (f.size() < need) return fail(err, "disk index truncated: pages missing");
  return true;
}

// Reads sectors 1..num_pages into dst (num_pages * 4096 bytes), as
// src/pure_mem.cu:45-69 does.
inline bool read_disk_pages(const std::string& path, const DiskLayout& L, void* dst,
                            std::string* err) {
  File f(path, "rb");
  if (!f) return fail(err, "cannot open index file " + path);
  if (!f.seek(kSectorBytes)) return fail(err, "seek failed in " + path);
  uint8_t* p = (uint8_t*)dst;
  int64_t total = L.num_pages * kSectorBytes;
  const int64_t chunk = int64_t(256) << 20;
  for (int64_t off = 0; off < total; off += chunk) {
    int64_t n = total - off < chunk ? total - off : chunk;
    if (!f.read(p + off, (size_t)n)) return fail(err, "short read of index pages");
  }
  return true;
}

// Writes a disk index.  coords: [n][dim] of elem_size bytes; adjacency: CSR
// (offsets [n+1], ids).  R = max degree slot count.  Sector 0 carries nr = 9
// values (the 8 read by the reference plus the file size, as upstream DiskANN).
inline bool write_disk_index(const std::string& path, int64_t n, int64_t dim, int64_t elem_size,
                             int64_t R, int64_t medoid, const void* coords,
                             const int64_t* adj_off, const uint32_t* adj_ids, std::string* err) {
  int64_t data_len = dim * elem_size;
  int64_t node_len = data_len + 4 * (R + 1);
  if (node_len > kSectorBytes) return fail(err, "node record larger than a sector");
  int64_t npp = kSectorBytes / node_len;
  int64_t pages = (n + npp - 1) / npp;
  File f(path, "wb");
  if (!f) return fail(err, "cannot create " + path);
  std::vector<uint8_t> sector(kSectorBytes, 0);
  uint32_t nr_nc[2] = {9, 1};
  uint64_t meta[9] = {(uint64_t)n, (uint64_t)dim, (uint64_t)medoid, (uint64_t)node_len,
                      (uint64_t)npp, 0, 0, 0, (uint64_t)((pages + 1) * kSectorBytes)};
  std::memcpy(sector.data(), nr_nc, sizeof(nr_nc));
  std::memcpy(sector.data() + sizeof(nr_nc), meta, sizeof(meta));
  if (!f.write(sector.data(), sector.size())) return fail(err, "write failed: " + path);
  const uint8_t* c = (const uint8_t*)coords;
  for (int64_t p = 0; p < pages; ++p) {
    std::fill(sector.begin(), sector.end(), 0);
    for (int64_t s = 0; s < npp; ++s) {
      int64_t u = p * npp + s;
      if (u >= n) break;
      uint8_t* rec = sector.data() + s * node_len;
      std::memcpy(rec, c + u * data_len, (size_t)data_len);
      int64_t deg = adj_off[u + 1] - adj_off[u];
      if (deg > R) return fail(err, "adjacency list longer than R");
      uint32_t d32 = (uint32_t)deg;
      std::memcpy(rec + data_len, &d32, 4);
      std::memcpy(rec + data_len + 4, adj_ids + adj_off[u], (size_t)deg * 4);
    }
    if (!f.write(sector.data(), sector.size())) return fail(err, "write failed: " + path);
  }
  return true;
}

// ---------------------------------------------------------------- PQ

inline bool read_pq(const std::string& pivots_path, const std::string& codes_path, PQHost* pq,
                    bool load_codes, std::string* err) {
  int32_t nr = 0, nc = 0;
  std::vector<uint64_t> offs;
  if (!read_bin(pivots_path, 0, &nr, &nc, &offs, err)) return false;
  if (!((nr == 4 || nr == 5) && nc == 1))  // src/pq_search.cu:79-81
    return fail(err, "pq pivots: offset table must be 4x1 or 5x1");
  bool legacy = nr == 5;
  int32_t a = 0, b = 0;
  if (!read_bin(pivots_path, (int64_t)offs[0], &a, &b, &pq->pivots, err)) return false;
  if (a != kNumPivots) return fail(err, "pq pivots: expected 256 centroids");  // :87
  pq->dim = b;
  if (!read_bin(pivots_path, (int64_t)offs[1], &a, &b, &pq->centroid, err)) return false;
  if (a != pq->dim || b != 1) return fail(err, "pq centroid: shape mismatch");  // :96
  int chunk_idx = legacy ? 3 : 2;  // src/pq_search.cu:103
  if (!read_bin(pivots_path, (int64_t)offs[chunk_idx], &a, &b, &pq->chunk_offsets, err))
    return false;
  if (b != 1 || a < 2) return fail(err, "pq chunk offsets: shape mismatch");
  pq->num_chunks = a - 1;
  // The reference maps each dim to a chunk through these offsets
  // (src/pq_search.cu:111-117); a dim outside every chunk would index the
  // LUT out of range, so the offsets must tile [0, dim).
  if (pq->chunk_offsets[0] != 0 || pq->chunk_offsets[pq->num_chunks] != pq->dim)
    return fail(err, "pq chunk offsets must start at 0 and end at dim");
  for (int m = 0; m < pq->num_chunks; ++m)
    if (pq->chunk_offsets[m + 1] < pq->chunk_offsets[m])
      return fail(err, "pq chunk offsets must be non-decreasing");
  if (load_codes) {
    int32_t n = 0, m = 0;
    if (!read_bin(codes_path, 0, &n, &m, &pq->codes, err)) return false;
    if (m != pq->num_chunks)
      return fail(err, "pq compressed: chunk count differs from the pivots file");
    pq->num_pts = n;
  } else {
    File f(codes_path, "rb");
    if (!f) return fail(err, "cannot open " + codes_path);
    int32_t hdr[2];
    if (!f.read(hdr, sizeof(hdr))) return fail(err, "truncated " + codes_path);
    pq->num_pts = hdr[0];
  }
  return true;
}

inline bool write_pq(const std::string& pivots_path, const std::string& codes_path,
                     const PQHost& pq, std::string* err) {
  {
    File f(pivots_path, "wb");
    if (!f) return fail(err, "cannot create " + pivots_path);
    uint64_t offs[4];
    offs[0] = (uint64_t)kSectorBytes;
    int64_t w = write_bin_at(f, (int64_t)offs[0], kNumPivots, pq.dim, pq.pivots.data(), 4);
    if (w < 0) return fail(err, "write failed: " + pivots_path);
    offs[1] = offs[0] + (uint64_t)w;
    w = write_bin_at(f, (int64_t)offs[1], pq.dim, 1, pq.centroid.data(), 4);
    if (w < 0) return fail(err, "write failed: " + pivots_path);
    offs[2] = offs[1] + (uint64_t)w;
    w = write_bin_at(f, (int64_t)offs[2], pq.num_chunks + 1, 1, pq.chunk_offsets.data(), 4);
    if (w < 0) return fail(err, "write failed: " + pivots_path);
    offs[3] = offs[2] + (uint64_t)w;
    if (write_bin_at(f, 0, 4, 1, offs, 8) < 0) return fail(err, "write failed: " + pivots_path);
  }
  return write_bin(codes_path, (int32_t)pq.num_pts, pq.num_chunks, pq.codes.data(), 1, err);
}

// ---------------------------------------------------------------- nav graph

inline bool read_nav(const std::string& prefix, int64_t elem_size, NavHost* nav,
                     std::string* err) {
  const std::string idx_path = prefix + "/nav_index";
  const std::string data_path = prefix + "/nav_index.data";
  const std::string map_path = prefix + "/map.txt";
  int32_t n = 0, d = 0;
  if (!read_bin_raw(data_path, 0, (size_t)elem_size, &n, &d, &nav->data, err)) return false;
  if (n <= 0 || d <= 0) return fail(err, "nav_index.data: empty");
  nav->num_node = n;
  nav->dim = d;
  {
    File f(map_path, "r");
    if (!f) return fail(err, "cannot open " + map_path);
    nav->mapping.resize((size_t)n);
    for (int32_t i = 0; i < n; ++i) {
      int x;
      if (std::fscanf(f.get(), "%d", &x) != 1) return fail(err, "map.txt: too few entries");
      nav->mapping[(size_t)i] = x;
    }
  }
  File f(idx_path, "rb");
  if (!f) return fail(err, "cannot open " + idx_path);
  uint64_t file_size = 0, frozen = 0;
  uint32_t max_m = 0, start = 0;
  if (!f.read(&file_size, 8) || !f.read(&max_m, 4) || !f.read(&start, 4) || !f.read(&frozen, 8))
    return fail(err, "nav_index: truncated header");
  // src/nav_graph.cu:86 asserts 0 < max_m <= 32.
  if (max_m == 0 || max_m > 32) return fail(err, "nav_index: max degree must be in [1, 32]");
  if ((int64_t)start >= nav->num_node) return fail(err, "nav_index: start out of range");
  nav->max_m = (int)max_m;
  nav->start = (int)start;
  nav->graph.assign((size_t)n * max_m, -1);
  for (int32_t i = 0; i < n; ++i) {
    uint32_t k = 0;
    if (!f.read(&k, 4)) return fail(err, "nav_index: truncated adjacency");
    if (k == 0 || k > max_m) return fail(err, "nav_index: node degree must be in [1, max_m]");  // :90
    if (!f.read(nav->graph.data() + (size_t)i * max_m, (size_t)k * 4))
      return fail(err, "nav_index: truncated adjacency");
    for (uint32_t j = 0; j < k; ++j) {
      int32_t v = nav->graph[(size_t)i * max_m + j];
      if (v < 0 || v >= n) return fail(err, "nav_index: neighbour id out of range");
    }
  }
  return true;
}

inline bool write_nav(const std::string& prefix, const NavHost& nav, int64_t elem_size,
                      const std::vector<int64_t>& adj_off, const std::vector<uint32_t>& adj_ids,
                      std::string* err) {
  if (!write_bin(prefix + "/nav_index.data", (int32_t)nav.num_node, nav.dim, nav.data.data(),
                 (size_t)elem_size, err))
    return false;
  {
    File f(prefix + "/map.txt", "w");
    if (!f) return fail(err, "cannot create map.txt");
    for (int64_t i = 0; i < nav.num_node; ++i) std::fprintf(f.get(), "%d\n", nav.mapping[(size_t)i]);
  }
  File f(prefix + "/nav_index", "wb");
  if (!f) return fail(err, "cannot create nav_index");
  uint32_t max_deg = 0;
  for (int64_t i = 0; i < nav.num_node; ++i) {
    uint32_t k = (uint32_t)(adj_off[(size_t)i + 1] - adj_off[(size_t)i]);
    if (k > max_deg) max_deg = k;
  }
  uint64_t file_size = 24 + 4 * (uint64_t)nav.num_node + 4 * (uint64_t)adj_ids.size();
  uint64_t frozen = 0;
  uint32_t start = (uint32_t)nav.start;
  if (!f.write(&file_size, 8) || !f.write(&max_deg, 4) || !f.write(&start, 4) || !f.write(&frozen, 8))
    return fail(err, "write failed: nav_index");
  for (int64_t i = 0; i < nav.num_node; ++i) {
    uint32_t k = (uint32_t)(adj_off[(size_t)i + 1] - adj_off[(size_t)i]);
    if (!f.write(&k, 4) || !f.write(adj_ids.data() + adj_off[(size_t)i], (size_t)k * 4))
      return fail(err, "write failed: nav_index");
  }
  return true;
}

// ---------------------------------------------------------------- *vecs

// Reads bvecs/fvecs/ivecs (elem = 1 or 4); rows must share one dimension.
inline bool read_vecs(const std::string& path, size_t elem, int64_t* n_out, int64_t* d_out,
                      std::vector<uint8_t>* out, std::string* err) {
  File f(path, "rb");
  if (!f) return fail(err, "cannot open " + path);
  int32_t d = 0;
  if (!f.read(&d, 4)) return fail(err, "empty vecs file " + path);
  if (d <= 0 || d >= 1000000) return fail(err, "unreasonable dimension in " + path);
  int64_t sz = f.size();
  int64_t row = 4 + (int64_t)d * (int64_t)elem;
  if (sz % row != 0) return fail(err, "weird file size for " + path);
  int64_t n = sz / row;
  out->resize((size_t)(n * d * (int64_t)elem));
  f.seek(0);
  std::vector<uint8_t> buf((size_t)row);
  for (int64_t i = 0; i < n; ++i) {
    if (!f.read(buf.data(), buf.size())) return fail(err, "short read in " + path);
    int32_t di;
    std::memcpy(&di, buf.data(), 4);
    if (di != d) return fail(err, "inconsistent row dimension in " + path);
    std::memcpy(out->data() + (size_t)(i * d * (int64_t)elem), buf.data() + 4, (size_t)(d * (int64_t)elem));
  }
  *n_out = n;
  *d_out = d;
  return true;
}

inline bool write_vecs(const std::string& path, size_t elem, int64_t n, int64_t d,
                       const void* data, std::string* err) {
  File f(path, "wb");
  if (!f) return fail(err, "cannot create " + path);
  const uint8_t* p = (const uint8_t*)data;
  int32_t d32 = (int32_t)d;
  for (int64_t i = 0; i < n; ++i) {
    if (!f.write(&d32, 4) || !f.write(p + (size_t)(i * d * (int64_t)elem), (size_t)(d * (int64_t)elem)))
      return fail(err, "write failed: " + path);
  }
  return true;
}

}  // namespace gann
