// search_mem: command line of the in-memory search, compatible with the
// reference's `search_mem` (bin/search_disk.cpp built with -DUSE_PURE_MEM,
// bin/CMakeLists.txt:34-41): same flags, same query replication, same
// result lines and L-sweep table, on top of the C ABI of libgustann_hip.so.
//
//   search_mem --query Q --index I --pq_data P [--nav_graph N] --data_type uint8|float
//              [--ground_truth GT] [--topk K] --ef_search L [L ...] [-R n] [-G]
//              [--mode fused|gp|lut|stepwise|paged|uring] [--beam_width W] [--device d]
//              [--result_path FILE]
//
// Additions: --mode selects the execution mode (GANN_MODE_*), --beam_width
// the beam search of this library (1, the default, is the reference's one
// node per iteration; 2..4 expand that many list entries per round), and
// --result_path writes the ids of the first L's run as a bin file
// [nq x topk] int32, the input of check_recall.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>
#include <string>
#include <vector>

#include "formats.hpp"
#include "gustann.h"

namespace {

[[noreturn]] void die(const std::string& msg) {
  std::fprintf(stderr, "%s\n", msg.c_str());
  std::exit(1);
}

void check(int rc, const char* what) {
  if (rc != GANN_OK) die(std::string(what) + " failed: " + gann_last_error());
}

// calc_recall (bin/utils.hpp:104-116): the fraction is formed in double and
// returned as float, which the caller prints as double.
float calc_recall(const int32_t* res, const int32_t* gt, int64_t num, int64_t dim, int k) {
  int64_t cnt = 0;
  for (int64_t i = 0; i < num; ++i) {
    std::set<int32_t> s(gt + i * dim, gt + i * dim + k);
    for (int j = 0; j < k; ++j)
      if (s.count(res[i * k + j])) ++cnt;
  }
  return (float)(1.0 * (double)cnt / (double)(num * k));
}

void usage() {
  std::fprintf(stderr,
               "Usage: search_mem --query FILE --index FILE --pq_data PREFIX --data_type uint8|float\n"
               "                  --ef_search L [L ...] [--ground_truth FILE] [--topk K]\n"
               "                  [--nav_graph DIR] [--repeat|-R N] [--use-gpu-mem|-G]\n"
               "                  [--mode fused|gp|lut|stepwise|paged|uring] [--beam_width W]\n"
               "                  [--device D] [--result_path FILE]\n");
}

}  // namespace

int main(int argc, char** argv) {
  std::string query_file, index_file, gt_file, data_type, pq_prefix, nav_prefix, mode_s = "fused";
  std::string result_path;
  int topk = 100;  // bin/search_disk.cpp:29
  int repeat = 20; // :36
  int device = 0;
  int beam_width = 1;
  bool use_gpu_mem = false;
  std::vector<int> ef;
  for (int i = 1; i < argc; ++i) {
    std::string a = argv[i];
    auto need = [&](const char* name) -> std::string {
      if (i + 1 >= argc) die(std::string("missing value for ") + name);
      return argv[++i];
    };
    if (a == "--query") query_file = need("--query");
    else if (a == "--index") index_file = need("--index");
    else if (a == "--ground_truth") gt_file = need("--ground_truth");
    else if (a == "--data_type") data_type = need("--data_type");
    else if (a == "--topk") topk = std::atoi(need("--topk").c_str());
    else if (a == "--pq_data") pq_prefix = need("--pq_data");
    else if (a == "--nav_graph") nav_prefix = need("--nav_graph");
    else if (a == "--repeat" || a == "-R") repeat = std::atoi(need("--repeat").c_str());
    else if (a == "--use-gpu-mem" || a == "-G") use_gpu_mem = true;
    else if (a == "--mode") mode_s = need("--mode");
    else if (a == "--device") device = std::atoi(need("--device").c_str());
    else if (a == "--beam_width") beam_width = std::atoi(need("--beam_width").c_str());
    else if (a == "--result_path") result_path = need("--result_path");
    else if (a == "--ef_search") {
      while (i + 1 < argc && argv[i + 1][0] != '-') ef.push_back(std::atoi(argv[++i]));
    } else if (a == "-h" || a == "--help") {
      usage();
      return 0;
    } else {
      usage();
      die("unknown argument " + a);
    }
  }
  if (query_file.empty() || index_file.empty() || data_type.empty() || pq_prefix.empty()) {
    usage();
    die("--query, --index, --data_type and --pq_data are required");
  }
  int dtype;
  if (data_type == "float") dtype = GANN_FLOAT;
  else if (data_type == "uint8") dtype = GANN_UINT8;
  else die("unrecognized data type " + data_type);
  int mode = GANN_MODE_FUSED;
  if (mode_s == "lut") mode = GANN_MODE_FUSED_LUT;
  else if (mode_s == "gp") mode = GANN_MODE_FUSED_GP;
  else if (mode_s == "stepwise") mode = GANN_MODE_STEPWISE;
  else if (mode_s == "paged") mode = GANN_MODE_STEPWISE_PAGED;
  else if (mode_s == "uring") mode = GANN_MODE_STEPWISE_URING;
  else if (mode_s != "fused") die("unknown --mode " + mode_s);
  if (beam_width < 1) die("--beam_width must be >= 1 (1 = the reference's one node per iteration)");
  if (ef.empty()) die("--ef_search needs at least one value");
  for (int L : ef)
    if (L < topk) die("ef_search must be >= topk (bin/search_disk.cpp:189-192)");
  if (repeat < 1) die("--repeat must be >= 1");

  std::printf("%s\n", gann_version());
  gann_config cfg{index_file.c_str(), pq_prefix.c_str(), nav_prefix.empty() ? nullptr : nav_prefix.c_str(),
                  dtype, use_gpu_mem ? GANN_PLACEMENT_HBM : GANN_PLACEMENT_HOST_PINNED, device};
  gann_handle* h = nullptr;
  check(gann_open(&cfg, &h), "gann_open");
  gann_index_info info{};
  check(gann_get_info(h, &info), "gann_get_info");

  // queries: uint8 bvecs converted to float, or fvecs (bin/search_disk.cpp:152-167)
  std::string err;
  int64_t nq = 0, d = 0;
  std::vector<uint8_t> raw;
  if (!gann::read_vecs(query_file, dtype == GANN_UINT8 ? 1 : 4, &nq, &d, &raw, &err)) die(err);
  if (d != info.dim) die("query dimension differs from the index");
  std::vector<float> q((size_t)(nq * d));
  if (dtype == GANN_UINT8)
    for (size_t i = 0; i < q.size(); ++i) q[i] = (float)raw[i];
  else
    std::memcpy(q.data(), raw.data(), q.size() * 4);
  std::printf("Read %lld queries\n", (long long)nq);
  // replicate repeat times (:172-183)
  const int64_t total = nq * repeat;
  std::vector<float> qr((size_t)(total * d));
  for (int r = 0; r < repeat; ++r) std::memcpy(qr.data() + (size_t)(r * nq * d), q.data(), q.size() * 4);
  std::vector<int32_t> nns((size_t)(total * topk)), found((size_t)total);
  std::vector<float> dis((size_t)(total * topk));

  std::vector<uint8_t> gt_raw;
  int64_t gt_nq = 0, gt_d = 0;
  const bool have_gt = !gt_file.empty();
  if (have_gt && !gann::read_vecs(gt_file, 4, &gt_nq, &gt_d, &gt_raw, &err)) die(err);
  const int32_t* gt = reinterpret_cast<const int32_t*>(gt_raw.data());
  if (have_gt && gt_nq > total) die("ground truth has more rows than queries");

  auto run = [&](int L, gann_stats* st) {
    check(gann_search_ex(h, qr.data(), (int32_t)total, topk, L, beam_width, mode, nns.data(), dis.data(),
                         found.data(), nullptr, st),
          "gann_search");
  };
  auto save = [&]() {
    if (result_path.empty()) return;
    if (!gann::write_bin(result_path, (int32_t)total, topk, nns.data(), 4, &err)) die(err);
  };
  if (ef.size() == 1) {
    gann_stats st{};
    run(ef[0], &st);
    save();
    for (int i = 0; i < 5 && i < total; ++i) {  // :199-204
      for (int j = 0; j < 5 && j < topk; ++j) std::printf("%lf(%d)\t", dis[(size_t)(i * topk + j)], nns[(size_t)(i * topk + j)]);
      std::printf("\n");
    }
    std::printf("Run time: %lf s, QPS: %.2f\n", st.run_time_s, total / st.run_time_s);
    if (have_gt) {
      if (topk > gt_d) die("topk exceeds the ground-truth width");
      double recall = calc_recall(nns.data(), gt, gt_nq, gt_d, topk);
      std::printf("Recall @ %d: %lf\n", topk, recall);
      std::printf("[REPORT] RECALL: %lf\n", recall);
    }
  } else {
    struct Row {
      int L;
      double qps, recall;
    };
    std::vector<Row> rows;
    for (int L : ef) {
      gann_stats st{};
      run(L, &st);
      if (L == ef[0]) save();
      rows.push_back({L, total / st.run_time_s,
                      (have_gt && topk <= gt_d) ? calc_recall(nns.data(), gt, gt_nq, gt_d, topk) : -1});
    }
    std::string header = have_gt ? "Recall@" + std::to_string(topk) : "Recall";
    std::printf("\n%-12s %-18s %-18s %-18s\n", "L", "Run Time (s)", "QPS", header.c_str());
    std::printf("%-12s %-18s %-18s %-18s\n", "------------", "------------------",
                "------------------", "------------------");
    for (const Row& r : rows) {
      if (r.recall >= 0)
        std::printf("%-12d %-18.6f %-18.2f %-18.6f\n", r.L, total / r.qps, r.qps, r.recall);
      else
        std::printf("%-12d %-18.6f %-18.2f %-18s\n", r.L, total / r.qps, r.qps, "N/A");
    }
  }
  check(gann_close(h), "gann_close");
  return 0;
}
