// gustann.hpp — header-only C++ facade with the reference's class interface
// over the C ABI of include/gustann.h, so code written against
// gustann::GustANN (src/ssd_search.hpp:29-83) compiles unchanged for the
// in-memory executor.  Errors surface as gustann::Error (a
// std::runtime_error carrying the C status code) where the reference
// aborted, exited or threw.
#pragma once

#include <stdexcept>
#include <string>

#include "gustann.h"

namespace gustann {

// src/common.hpp:22-25
enum DataType { UINT8 = GANN_UINT8, FLOAT = GANN_FLOAT };

// src/ssd_search.hpp:18-23
class GustANNConfig {
 public:
  std::string index_file;
  std::string pq_file_prefix;
  std::string nav_graph_prefix;
};

// src/ssd_search.hpp:25-27 (run_time) plus the device counters
struct GustANNStats {
  double run_time = 0;
  double entry_time = 0;
  long long n_expansions = 0;
  long long n_adc = 0;
  double alg_bytes = 0;
  long long n_nav_fallback = 0;
};

class Error : public std::runtime_error {
 public:
  Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

inline void check(int rc) {
  if (rc != GANN_OK) throw Error(rc, gann_last_error());
}

class GustANN {
 public:
  explicit GustANN(DataType data_type = FLOAT, int device_id = 0)
      : data_type_(data_type), device_id_(device_id) {}
  GustANN(const GustANN&) = delete;
  GustANN& operator=(const GustANN&) = delete;
  ~GustANN() {
    if (h_) gann_close(h_);
  }

  // src/ssd_search.cu:108-112
  void init_pure_mem(const GustANNConfig& cfg, bool use_gpu_mem) {
    if (h_) {
      gann_close(h_);
      h_ = nullptr;
    }
    gann_config c{cfg.index_file.c_str(), cfg.pq_file_prefix.c_str(),
                  cfg.nav_graph_prefix.empty() ? nullptr : cfg.nav_graph_prefix.c_str(),
                  (int32_t)data_type_,
                  use_gpu_mem ? GANN_PLACEMENT_HBM : GANN_PLACEMENT_HOST_PINNED, device_id_};
    check(gann_open(&c, &h_));
  }

  // src/ssd_search.cu:114-140
  void search(const float* qdata, int num_queries, int topk, int ef_search, int* nns,
              float* distances, int* found_cnt, GustANNStats* stats = nullptr) {
    if (!h_) throw Error(GANN_ERR_INVALID, "UnInited! (src/ssd_search.cu:138-139)");
    gann_stats st{};
    check(gann_search(h_, qdata, num_queries, topk, ef_search, 1, nns, distances, found_cnt, &st));
    if (stats) {
      stats->run_time = st.run_time_s;
      stats->entry_time = st.entry_time_s;
      stats->n_expansions = st.n_expansions;
      stats->n_adc = st.n_adc;
      stats->alg_bytes = st.alg_bytes;
      stats->n_nav_fallback = st.n_nav_fallback;
    }
  }

  gann_handle* handle() const { return h_; }

 private:
  DataType data_type_;
  int device_id_;
  gann_handle* h_ = nullptr;
};

}  // namespace gustann
