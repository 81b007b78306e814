// TEST INFRASTRUCTURE ONLY — a C-ABI shim around the reference's own C++.
//
// This file is compiled together with the reference sources where they lie
// under /root/reference/cpp (soap.cpp, neighbor_list.cpp, neighbor.cpp,
// control.cpp; see
// oracle/Makefile).  It only forwards flat arrays to
//   mdescriptor::SoapCalculator::compute   (cpp/src/standalone/soap.cpp:1254-1258)
//   mdescriptor::build_neighbor_graph      (cpp/src/common/neighbor.cpp:703-768)
//   mdescriptor::compute_neighbor_list     (cpp/src/standalone/neighbor_list.cpp:15-78)
// so that tests can check the oracle restatement, and bench.py can time the
// reference CPU path ("cpu_baseline.kind = reference").  The built library
// lands in oracle/_ref/ and is never part of the product.
#include "mdescriptor/descriptor.hpp"
#include "mdescriptor/local_descriptors.hpp"
#include "mdescriptor/neighbor.hpp"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <vector>

namespace {

void copy_error(char* err, int errlen, const char* message) {
    if (err != nullptr && errlen > 0) {
        std::snprintf(err, static_cast<std::size_t>(errlen), "%s", message);
    }
}

mdescriptor::StructureBatchView view(const std::int32_t* numbers, const double* positions,
                                     const double* cells, const std::int32_t* pbc,
                                     const std::int64_t* offsets, std::int64_t structures,
                                     std::int64_t atoms) {
    mdescriptor::StructureBatchView batch;
    batch.numbers = numbers;
    batch.positions = positions;
    batch.cells = cells;
    batch.pbc = pbc;
    batch.offsets = offsets;
    batch.structures = structures;
    batch.atoms = atoms;
    return batch;
}

} // namespace

extern "C" {

// The SoapOptions fields beyond the GTO, uncompressed, unweighted default
// (same layout as the oracle's mdxo_soap_options).
struct mdxr_soap_options {
    std::int32_t weighting_function; // 0 none, 1 poly, 2 pow, 3 exp
    std::int32_t weighting_has_w0;
    double weighting_r0, weighting_c, weighting_d, weighting_m, weighting_w0;
    const double* species_weights; // n_species values or null (all 1)
    std::int32_t compression;      // 0 off, 1 mu2, 2 mu1nu1, 3 crossover
    std::int32_t radial_basis;     // 0 GTO, 1 polynomial
    std::int32_t grid_size;
    const double* radial_grid;
    const double* radial_weights;
    const double* radial_values;   // n_max x grid_size
};

// SOAP with the option mapping of SoapKernel._ensure_native (core.py:229-270);
// opt may be null (rbf = "gto", compression "off", default weighting).
// average: 0 off, 1 inner, 2 outer.  Returns 0, 1 (invalid) or 4 (cancelled).
int mdxr_soap(const std::int32_t* numbers, const double* positions, const double* cells,
              const std::int32_t* pbc, const std::int64_t* offsets, std::int64_t structures,
              std::int64_t atoms, const std::int32_t* species, int n_species, int n_max, int l_max,
              double r_cut, double sigma, const double* alphas, const double* betas,
              const mdxr_soap_options* opt, int average, int num_threads, double* output, char* err,
              int errlen) {
    try {
        mdescriptor::SoapOptions options;
        options.species.assign(species, species + n_species);
        options.r_cut = r_cut;
        options.n_max = n_max;
        options.l_max = l_max;
        options.sigma = sigma;
        const bool polynomial = opt != nullptr && opt->radial_basis == 1;
        options.radial_basis = polynomial ? 1 : 0;
        if (polynomial) {
            const std::size_t q = static_cast<std::size_t>(opt->grid_size);
            options.radial_grid.assign(opt->radial_grid, opt->radial_grid + q);
            options.radial_weights.assign(opt->radial_weights, opt->radial_weights + q);
            options.radial_values.assign(opt->radial_values,
                                         opt->radial_values + q * static_cast<std::size_t>(n_max));
        } else {
            const std::size_t radial = static_cast<std::size_t>(l_max + 1) * static_cast<std::size_t>(n_max);
            options.alphas.assign(alphas, alphas + radial);
            options.betas.assign(betas, betas + radial * static_cast<std::size_t>(n_max));
        }
        if (opt != nullptr && opt->species_weights != nullptr) {
            options.species_weights.assign(opt->species_weights, opt->species_weights + n_species);
        } else {
            options.species_weights.assign(static_cast<std::size_t>(n_species), 1.0);
        }
        if (opt != nullptr) {
            options.weighting_has_function = opt->weighting_function != 0;
            options.weighting_function = opt->weighting_function;
            options.weighting_has_w0 = opt->weighting_has_w0 != 0;
            options.weighting_r0 = opt->weighting_r0;
            options.weighting_c = opt->weighting_c;
            options.weighting_d = opt->weighting_d;
            options.weighting_m = opt->weighting_m;
            options.weighting_w0 = opt->weighting_w0;
        }
        options.compression = opt != nullptr ? opt->compression : 0;
        options.inner_average = average == 1;
        options.outer_average = average == 2;
        options.num_threads = num_threads;
        mdescriptor::SoapCalculator calculator(std::move(options));
        calculator.compute(view(numbers, positions, cells, pbc, offsets, structures, atoms), output,
                           nullptr);
        return 0;
    } catch (const mdescriptor::CancelledError& exc) {
        copy_error(err, errlen, exc.what());
        return 4;
    } catch (const std::exception& exc) {
        copy_error(err, errlen, exc.what());
        return 1;
    }
}

struct mdxr_graph {
    std::int64_t atoms;
    std::int64_t pairs;
    std::int64_t* offsets;
    std::int32_t* neighbors;
    std::int32_t* shifts;
    double* displacements;
    double* distance2;
};

// build_neighbor_graph at `cutoff`, include_boundary as given, shifts stored.
int mdxr_graph_build(const std::int32_t* numbers, const double* positions, const double* cells,
                     const std::int32_t* pbc, const std::int64_t* offsets, std::int64_t structures,
                     std::int64_t atoms, double cutoff, int include_boundary, int num_threads,
                     mdxr_graph* out, char* err, int errlen) {
    std::memset(out, 0, sizeof(*out));
    try {
        const mdescriptor::NeighborGraph graph = mdescriptor::build_neighbor_graph(
            view(numbers, positions, cells, pbc, offsets, structures, atoms), cutoff, nullptr,
            num_threads, include_boundary != 0, false, true);
        const auto& o = graph.offsets();
        out->atoms = static_cast<std::int64_t>(o.size()) - 1;
        out->pairs = o.empty() ? 0 : o.back();
        const std::size_t p = static_cast<std::size_t>(out->pairs);
        out->offsets = new std::int64_t[o.size()];
        std::memcpy(out->offsets, o.data(), o.size() * sizeof(std::int64_t));
        out->neighbors = new std::int32_t[p + 1];
        out->shifts = new std::int32_t[3 * p + 1];
        out->displacements = new double[3 * p + 1];
        out->distance2 = new double[p + 1];
        if (p > 0) {
            std::memcpy(out->neighbors, graph.atoms_data().data(), p * sizeof(std::int32_t));
            std::memcpy(out->shifts, graph.shifts().data(), 3 * p * sizeof(std::int32_t));
            std::memcpy(out->displacements, graph.displacements().data(), 3 * p * sizeof(double));
            std::memcpy(out->distance2, graph.distance2().data(), p * sizeof(double));
        }
        return 0;
    } catch (const std::exception& exc) {
        copy_error(err, errlen, exc.what());
        return 1;
    }
}

void mdxr_graph_free(mdxr_graph* graph) {
    delete[] graph->offsets;
    delete[] graph->neighbors;
    delete[] graph->shifts;
    delete[] graph->displacements;
    delete[] graph->distance2;
    std::memset(graph, 0, sizeof(*graph));
}

struct mdxr_pair_table {
    std::int64_t rows;
    std::int64_t structures;
    double* values;         // rows x 9
    std::int64_t* offsets;  // structures + 1
};

// compute_neighbor_list(batch, cutoff, full_neighbor_list, self_pairs, num_threads, nullptr).
int mdxr_neighbor_list(const std::int32_t* numbers, const double* positions, const double* cells,
                       const std::int32_t* pbc, const std::int64_t* offsets, std::int64_t structures,
                       std::int64_t atoms, double cutoff, int full_neighbor_list, int self_pairs,
                       int num_threads, mdxr_pair_table* out, char* err, int errlen) {
    std::memset(out, 0, sizeof(*out));
    try {
        const mdescriptor::DescriptorPairTable table = mdescriptor::compute_neighbor_list(
            view(numbers, positions, cells, pbc, offsets, structures, atoms), cutoff,
            full_neighbor_list != 0, self_pairs != 0, num_threads, nullptr);
        out->rows = static_cast<std::int64_t>(table.values.size() / 9);
        out->structures = static_cast<std::int64_t>(table.offsets.size()) - 1;
        out->values = new double[table.values.size() + 1];
        out->offsets = new std::int64_t[table.offsets.size() + 1];
        std::memcpy(out->values, table.values.data(), table.values.size() * sizeof(double));
        std::memcpy(out->offsets, table.offsets.data(), table.offsets.size() * sizeof(std::int64_t));
        return 0;
    } catch (const std::exception& exc) {
        copy_error(err, errlen, exc.what());
        return 1;
    }
}

void mdxr_pair_table_free(mdxr_pair_table* table) {
    delete[] table->values;
    delete[] table->offsets;
    std::memset(table, 0, sizeof(*table));
}

} // extern "C"
