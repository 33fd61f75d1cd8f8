// Weight initialisation (ref: src/CppNet/utils/init.cpp:15-130): same
// methods, limits and per-element draw order (row-major loop over (i,j)).
#include "CppNet/utils/init.hpp"

#include <cmath>
#include <random>
#include <stdexcept>

namespace CppNet
{
    namespace Utils
    {
        static std::mt19937& rng()
        {
            static std::mt19937 g(std::random_device{}());
            return g;
        }

        void set_seed(uint64_t seed) { rng().seed(static_cast<std::mt19937::result_type>(seed)); }
        uint64_t next_seed()
        {
            const uint64_t hi = rng()(), lo = rng()();
            return (hi << 32) | lo;
        }

        template <class Dist>
        static Tensor<float, 2> draw(int rows, int cols, Dist dist)
        {
            Tensor<float, 2> w(rows, cols);
            for (int i = 0; i < rows; ++i)
                for (int j = 0; j < cols; ++j) w(i, j) = dist(rng());
            return w;
        }

        Tensor<float, 2> xavier_uniform(int rows, int cols)
        {
            const float limit = std::sqrt(6.0f / static_cast<float>(rows + cols));
            return draw(rows, cols, std::uniform_real_distribution<float>(-limit, limit));
        }
        Tensor<float, 2> xavier_normal(int rows, int cols)
        {
            const float sd = std::sqrt(2.0f / static_cast<float>(rows + cols));
            return draw(rows, cols, std::normal_distribution<float>(0.0f, sd));
        }
        Tensor<float, 2> he_uniform(int rows, int cols)
        {
            const float limit = std::sqrt(6.0f / static_cast<float>(rows));
            return draw(rows, cols, std::uniform_real_distribution<float>(-limit, limit));
        }
        Tensor<float, 2> he_normal(int rows, int cols)
        {
            const float sd = std::sqrt(2.0f / static_cast<float>(rows));
            return draw(rows, cols, std::normal_distribution<float>(0.0f, sd));
        }
        Tensor<float, 2> uniform_init(int rows, int cols, float low, float high)
        {
            return draw(rows, cols, std::uniform_real_distribution<float>(low, high));
        }
        Tensor<float, 2> normal_init(int rows, int cols, float mean, float stddev)
        {
            return draw(rows, cols, std::normal_distribution<float>(mean, stddev));
        }
        Tensor<float, 2> constant_init(int rows, int cols, float value)
        {
            Tensor<float, 2> w(rows, cols);
            w.setConstant(value);
            return w;
        }
        Tensor<float, 2> init_weights(int rows, int cols, const std::string& method)
        {
            if (method == "xavier" || method == "glorot") return xavier_uniform(rows, cols);
            if (method == "xavier_normal" || method == "glorot_normal") return xavier_normal(rows, cols);
            if (method == "he" || method == "kaiming") return he_uniform(rows, cols);
            if (method == "he_normal" || method == "kaiming_normal") return he_normal(rows, cols);
            if (method == "uniform") return uniform_init(rows, cols);
            if (method == "normal") return normal_init(rows, cols);
            if (method == "zeros") return constant_init(rows, cols, 0.0f);
            if (method == "ones") return constant_init(rows, cols, 1.0f);
            throw std::invalid_argument("Unknown weight initialization method: " + method);
        }
    } // namespace Utils
} // namespace CppNet
