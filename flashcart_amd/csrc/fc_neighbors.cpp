// Host neighbour list (cell list over periodic images), the NeighborList.build
// replacement (reference src/flashcart/data/neighbors.py:56-77, :120-143).
//
// Output convention of the reference: pairs (i, j, S) with |pos[j] - pos[i] + S.cell| <
// cutoff, self pairs with S = 0 removed, and the edge list sorted by receiver i. The
// order inside a receiver block is not fixed by the reference (its backend does not
// document one); this library emits the canonical lexicographic order (i, j, Sx, Sy, Sz),
// so the result is a deterministic function of the inputs.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

struct Pair {
  int64_t i, j;
  int32_t s[3];
};

inline void cross(const double* a, const double* b, double* c) {
  c[0] = a[1] * b[2] - a[2] * b[1];
  c[1] = a[2] * b[0] - a[0] * b[2];
  c[2] = a[0] * b[1] - a[1] * b[0];
}

bool invert3(const double* m, double* inv) {
  const double det = m[0] * (m[4] * m[8] - m[5] * m[7]) - m[1] * (m[3] * m[8] - m[5] * m[6]) +
                     m[2] * (m[3] * m[7] - m[4] * m[6]);
  if (std::fabs(det) < 1e-300) return false;
  const double id = 1.0 / det;
  inv[0] = (m[4] * m[8] - m[5] * m[7]) * id;
  inv[1] = (m[2] * m[7] - m[1] * m[8]) * id;
  inv[2] = (m[1] * m[5] - m[2] * m[4]) * id;
  inv[3] = (m[5] * m[6] - m[3] * m[8]) * id;
  inv[4] = (m[0] * m[8] - m[2] * m[6]) * id;
  inv[5] = (m[2] * m[3] - m[0] * m[5]) * id;
  inv[6] = (m[3] * m[7] - m[4] * m[6]) * id;
  inv[7] = (m[1] * m[6] - m[0] * m[7]) * id;
  inv[8] = (m[0] * m[4] - m[1] * m[3]) * id;
  return true;
}

}  // namespace

// Returns the number of pairs (written only if <= capacity), or -1 for a singular cell,
// -2 for invalid arguments. cell: 3x3 row-major, rows are lattice vectors (pos = frac @ cell).
extern "C" int64_t fc_neighbor_list(int64_t n, const double* pos, const double* cell, const int32_t* pbc,
                                    double cutoff, int64_t capacity, int64_t* out_i, int64_t* out_j,
                                    int32_t* out_shift) {
  if (n < 0 || !(cutoff > 0.0)) return -2;
  if (n == 0) return 0;
  double inv[9];
  if (!invert3(cell, inv)) return -1;
  const double* a[3] = {cell, cell + 3, cell + 6};
  double vol_vec[3];
  cross(a[1], a[2], vol_vec);
  const double vol = std::fabs(a[0][0] * vol_vec[0] + a[0][1] * vol_vec[1] + a[0][2] * vol_vec[2]);
  // plane spacing h_k = V / |a_{k+1} x a_{k+2}|; fractional reach c_k = cutoff / h_k
  double reach[3];
  for (int k = 0; k < 3; ++k) {
    double c[3];
    cross(a[(k + 1) % 3], a[(k + 2) % 3], c);
    const double h = vol / std::sqrt(c[0] * c[0] + c[1] * c[1] + c[2] * c[2]);
    reach[k] = cutoff / h;
  }
  // wrapped fractional coordinates and integer offsets
  std::vector<double> w(3 * n);
  std::vector<int64_t> off(3 * n);
  double lo[3] = {0, 0, 0}, hi[3] = {1, 1, 1};
  for (int k = 0; k < 3; ++k)
    if (!pbc[k]) { lo[k] = 1e300; hi[k] = -1e300; }
  for (int64_t i = 0; i < n; ++i) {
    for (int k = 0; k < 3; ++k) {
      const double f = pos[3 * i] * inv[k] + pos[3 * i + 1] * inv[3 + k] + pos[3 * i + 2] * inv[6 + k];
      if (pbc[k]) {
        const double fl = std::floor(f);
        w[3 * i + k] = f - fl;
        off[3 * i + k] = (int64_t)fl;
      } else {
        w[3 * i + k] = f;
        off[3 * i + k] = 0;
        lo[k] = std::min(lo[k], f);
        hi[k] = std::max(hi[k], f);
      }
    }
  }
  // periodic images within reach of the home region
  int nimg[3];
  for (int k = 0; k < 3; ++k) nimg[k] = pbc[k] ? (int)std::ceil(reach[k]) : 0;
  struct Img { double f[3]; int64_t j; int32_t s[3]; };
  std::vector<Img> imgs;
  imgs.reserve((size_t)n * 2);
  for (int64_t j = 0; j < n; ++j)
    for (int sx = -nimg[0]; sx <= nimg[0]; ++sx)
      for (int sy = -nimg[1]; sy <= nimg[1]; ++sy)
        for (int sz = -nimg[2]; sz <= nimg[2]; ++sz) {
          const int s[3] = {sx, sy, sz};
          Img im;
          bool keep = true;
          for (int k = 0; k < 3; ++k) {
            im.f[k] = w[3 * j + k] + s[k];
            if (im.f[k] < lo[k] - reach[k] || im.f[k] > hi[k] + reach[k]) keep = false;
          }
          if (!keep) continue;
          im.j = j;
          for (int k = 0; k < 3; ++k) im.s[k] = s[k];
          imgs.push_back(im);
        }
  // bins of fractional width >= reach over [lo - reach, hi + reach]
  int nb[3];
  double base[3], width[3];
  for (int k = 0; k < 3; ++k) {
    base[k] = lo[k] - reach[k];
    const double span = (hi[k] + reach[k]) - base[k];
    nb[k] = std::max(1, (int)std::floor(span / reach[k]));
    nb[k] = std::min(nb[k], 512);
    width[k] = span / nb[k];
  }
  auto bin_of = [&](const double* f, int* b) {
    for (int k = 0; k < 3; ++k) {
      int v = (int)std::floor((f[k] - base[k]) / width[k]);
      b[k] = std::min(std::max(v, 0), nb[k] - 1);
    }
  };
  const int64_t nbins = (int64_t)nb[0] * nb[1] * nb[2];
  std::vector<int64_t> head(nbins + 1, 0), order(imgs.size());
  std::vector<int64_t> bid(imgs.size());
  for (size_t t = 0; t < imgs.size(); ++t) {
    int b[3];
    bin_of(imgs[t].f, b);
    bid[t] = ((int64_t)b[0] * nb[1] + b[1]) * nb[2] + b[2];
    head[bid[t] + 1]++;
  }
  for (int64_t b = 0; b < nbins; ++b) head[b + 1] += head[b];
  {
    std::vector<int64_t> fillp(head.begin(), head.end() - 1);
    for (size_t t = 0; t < imgs.size(); ++t) order[fillp[bid[t]]++] = (int64_t)t;
  }
  const double c2 = cutoff * cutoff;
  std::vector<Pair> pairs;
  std::vector<Pair> local;
  for (int64_t i = 0; i < n; ++i) {
    const double* fi = &w[3 * i];
    double xi[3];
    for (int k = 0; k < 3; ++k) xi[k] = fi[0] * cell[k] + fi[1] * cell[3 + k] + fi[2] * cell[6 + k];
    int b[3];
    bin_of(fi, b);
    local.clear();
    for (int dx = -1; dx <= 1; ++dx) {
      const int bx = b[0] + dx;
      if (bx < 0 || bx >= nb[0]) continue;
      for (int dy = -1; dy <= 1; ++dy) {
        const int by = b[1] + dy;
        if (by < 0 || by >= nb[1]) continue;
        for (int dz = -1; dz <= 1; ++dz) {
          const int bz = b[2] + dz;
          if (bz < 0 || bz >= nb[2]) continue;
          const int64_t bb = ((int64_t)bx * nb[1] + by) * nb[2] + bz;
          for (int64_t q = head[bb]; q < head[bb + 1]; ++q) {
            const Img& im = imgs[order[q]];
            double d2 = 0.0;
            for (int k = 0; k < 3; ++k) {
              const double xk = im.f[0] * cell[k] + im.f[1] * cell[3 + k] + im.f[2] * cell[6 + k];
              d2 += (xk - xi[k]) * (xk - xi[k]);
            }
            if (!(d2 < c2)) continue;
            Pair p;
            p.i = i;
            p.j = im.j;
            for (int k = 0; k < 3; ++k) p.s[k] = (int32_t)(im.s[k] - off[3 * im.j + k] + off[3 * i + k]);
            if (p.j == i && p.s[0] == 0 && p.s[1] == 0 && p.s[2] == 0) continue;
            local.push_back(p);
          }
        }
      }
    }
    std::sort(local.begin(), local.end(), [](const Pair& x, const Pair& y) {
      if (x.j != y.j) return x.j < y.j;
      if (x.s[0] != y.s[0]) return x.s[0] < y.s[0];
      if (x.s[1] != y.s[1]) return x.s[1] < y.s[1];
      return x.s[2] < y.s[2];
    });
    pairs.insert(pairs.end(), local.begin(), local.end());
  }
  const int64_t np = (int64_t)pairs.size();
  if (np <= capacity) {
    for (int64_t t = 0; t < np; ++t) {
      out_i[t] = pairs[t].i;
      out_j[t] = pairs[t].j;
      std::memcpy(out_shift + 3 * t, pairs[t].s, 3 * sizeof(int32_t));
    }
  }
  return np;
}
