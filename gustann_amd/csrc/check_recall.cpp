// check_recall: recall of a search result file against ground truth, with the
// interface and output of the reference's bin/check_recall.cpp:
//
//   check_recall OUTPUT_BIN GROUND_TRUTH_IVECS
//
// OUTPUT_BIN is a bin file (int32 npts, int32 ndims, then npts x ndims int32
// ids; bin/utils.hpp:91-101), e.g. written by `search_mem --result_path`.
// The ground truth is ivecs (bin/utils.hpp:55-57).  Prints
// "Recall @ k: r" with k = the result width, computed over every row as
// calc_recall (bin/utils.hpp:104-116).  The reference prints the dimensions
// in its row-count mismatch message; this one prints the row counts.
#include <cstdint>
#include <cstdlib>
#include <iostream>
#include <set>
#include <string>
#include <vector>

#include "formats.hpp"

namespace {

// calc_recall (bin/utils.hpp:104-116): the fraction is formed in double and
// returned as float.
float calc_recall(const int32_t* res, const int32_t* gt, int64_t num, int64_t dim, int64_t k) {
  int64_t cnt = 0;
  for (int64_t i = 0; i < num; ++i) {
    std::set<int32_t> s(gt + i * dim, gt + i * dim + k);
    for (int64_t j = 0; j < k; ++j)
      if (s.count(res[i * k + j])) ++cnt;
  }
  return (float)(1.0 * (double)cnt / (double)(num * k));
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    std::cout << argv[0] << ": output_bin ground_truth_bin" << std::endl;
    return -1;
  }
  std::string err;
  int64_t num = 0, dim = 0;
  std::vector<uint8_t> gt_raw;
  if (!gann::read_vecs(argv[2], 4, &num, &dim, &gt_raw, &err)) {
    std::cerr << err << std::endl;
    return -1;
  }
  int32_t num2 = 0, dim2 = 0;
  std::vector<int32_t> out;
  if (!gann::read_bin<int32_t>(argv[1], 0, &num2, &dim2, &out, &err)) {
    std::cerr << err << std::endl;
    return -1;
  }
  if (dim < dim2) {
    std::cout << "DIM mismatch: " << dim << " vs " << dim2 << std::endl;
    return -1;
  }
  if (num != num2) {
    std::cout << "NUM mismatch: " << num << " vs " << num2 << std::endl;
    return -1;
  }
  const int32_t* gt = reinterpret_cast<const int32_t*>(gt_raw.data());
  std::cout << "Recall @ " << dim2 << ": " << calc_recall(out.data(), gt, num, dim, dim2)
            << std::endl;
  return 0;
}
