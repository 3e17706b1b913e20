// A Net that runs on the host in double precision — TEST INFRASTRUCTURE.
//
// It executes each op of include/whispereacp/Net.h eagerly over host memory,
// with the arithmetic of the reference's scalar oracle (Tests/Decoder/
// Common.h:263-325, Tests/Encoder/Common.h:390-505): LayerNorm with the
// biased variance and eps 1e-5, exact GELU, attention scaled by
// 1/sqrt(head width) with query i of n standing at key position
// keyCount - n + i under the causal flag, embedding without sqrt(d). Weights
// are read from TensorBuffers placed with Device::host(); bindings are host
// ranges. The decoder body (DecoderRecording.cpp) records against it exactly
// as it does against HipNet, so the composition can be checked on a machine
// with no GPU.
#pragma once

#include <whispereacp/Net.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>

namespace WSP::Testing
{
class HostNet final : public Net
{
public:
    Tensor input(const Binding& source, const Shape& shape, DType type) override
    {
        const int r = shape.rank() == 1 ? shape[0] : shape.rows();
        const int c = shape.rank() == 1 ? 1 : shape.columns();
        if ((std::size_t) r * c * 4 > source.range.size)
            throw std::logic_error("input past its binding");
        Value v(r, c);
        for (int i = 0; i < r * c; ++i)
        {
            const char* at = static_cast<const char*>(source.range.data()) + 4 * (std::size_t) i;
            if (type == DType::int32)
            {
                std::int32_t x;
                std::memcpy(&x, at, 4);
                v.data[(std::size_t) i] = x;
            }
            else
            {
                float x;
                std::memcpy(&x, at, 4);
                v.data[(std::size_t) i] = x;
            }
        }
        return keep(std::move(v));
    }

    void output(const Tensor& value, const Binding& target) override
    {
        const Value& v = of(value);
        if (v.data.size() * 4 > target.range.size)
            throw std::logic_error("output past its binding");
        for (std::size_t i = 0; i < v.data.size(); ++i)
        {
            const float x = (float) v.data[i];
            std::memcpy(static_cast<char*>(target.range.data()) + 4 * i, &x, 4);
        }
    }

    Tensor rows(const Weight& table, int first, int count) override
    {
        const int c = table.dimension(1);
        Value v(count, c);
        for (int r = 0; r < count; ++r)
            for (int k = 0; k < c; ++k)
                v.at(r, k) = weightAt(table, (std::size_t) (first + r) * c + k);
        return keep(std::move(v));
    }

    Tensor transpose(const Tensor&) override { throw std::logic_error("transpose is not on the decoder's path"); }

    Tensor cached(const Cache& cache) override
    {
        const Storage& s = caches.at((std::size_t) cache.id);
        Value v(cache.rows, s.width);
        std::copy(s.data.begin(), s.data.begin() + (std::ptrdiff_t) cache.rows * s.width, v.data.begin());
        return keep(std::move(v));
    }

    Tensor conv1d(const Tensor&, const Weight&, const Weight&, int, int, Activation) override
    {
        throw std::logic_error("conv1d is not on the decoder's path");
    }

    Tensor linear(const Tensor& input, const Weight& weight, const Weight* bias, Activation activation) override
    {
        return keep(project(of(input), weight, bias, activation));
    }

    Tensor linearAdd(const Tensor& input, const Weight& weight, const Weight* bias, const Tensor& stream) override
    {
        Value y = project(of(input), weight, bias, Activation::none);
        const Value& s = of(stream);
        if (s.data.size() != y.data.size())
            throw std::logic_error("linearAdd: the stream and the projection differ in shape");
        for (std::size_t i = 0; i < y.data.size(); ++i)
            y.data[i] += s.data[i];
        return keep(std::move(y));
    }

    Tensor add(const Tensor& stream, const Tensor& addend) override
    {
        Value y = of(stream);
        const Value& a = of(addend);
        for (std::size_t i = 0; i < y.data.size(); ++i)
            y.data[i] += a.data[i];
        return keep(std::move(y));
    }

    Tensor layerNorm(const Tensor& input, const Weight& weight, const Weight& bias) override
    {
        const Value& x = of(input);
        Value y(x.rows, x.cols);
        for (int r = 0; r < x.rows; ++r)
        {
            double mean = 0, variance = 0;
            for (int c = 0; c < x.cols; ++c)
                mean += x.at(r, c);
            mean /= x.cols;
            for (int c = 0; c < x.cols; ++c)
                variance += (x.at(r, c) - mean) * (x.at(r, c) - mean);
            const double scale = 1.0 / std::sqrt(variance / x.cols + (double) 1e-5f);
            for (int c = 0; c < x.cols; ++c)
                y.at(r, c) = (x.at(r, c) - mean) * scale * weightAt(weight, (std::size_t) c) + weightAt(bias, (std::size_t) c);
        }
        return keep(std::move(y));
    }

    Tensor attention(const Tensor& queries, const Tensor& keys, const Tensor& values, int heads, bool causal) override
    {
        const Value &q = of(queries), &k = of(keys), &v = of(values);
        const int width = q.cols, hd = width / heads;
        const double scale = 1.0 / std::sqrt((double) hd);
        Value out(q.rows, width);
        std::vector<double> weights((std::size_t) k.rows);
        for (int h = 0; h < heads; ++h)
            for (int i = 0; i < q.rows; ++i)
            {
                const int last = causal ? k.rows - q.rows + i : k.rows - 1;
                double top = -INFINITY, sum = 0;
                for (int j = 0; j <= last; ++j)
                {
                    double dot = 0;
                    for (int c = 0; c < hd; ++c)
                        dot += q.at(i, h * hd + c) * k.at(j, h * hd + c);
                    weights[(std::size_t) j] = scale * dot;
                    top = std::max(top, weights[(std::size_t) j]);
                }
                for (int j = 0; j <= last; ++j)
                {
                    weights[(std::size_t) j] = std::exp(weights[(std::size_t) j] - top);
                    sum += weights[(std::size_t) j];
                }
                for (int c = 0; c < hd; ++c)
                {
                    double acc = 0;
                    for (int j = 0; j <= last; ++j)
                        acc += weights[(std::size_t) j] * v.at(j, h * hd + c);
                    out.at(i, h * hd + c) = acc / sum;
                }
            }
        return keep(std::move(out));
    }

    Tensor embed(const Tensor& tokens, const Weight& tokenTable, const Weight& positionTable, int firstPosition) override
    {
        const Value& t = of(tokens);
        const int n = t.rows * t.cols, width = tokenTable.dimension(1);
        Value y(n, width);
        for (int i = 0; i < n; ++i)
        {
            const long long id = (long long) t.data[(std::size_t) i];
            if (id < 0 || id >= tokenTable.dimension(0) || firstPosition + i >= positionTable.dimension(0))
                throw std::logic_error("embed outside its tables");
            for (int c = 0; c < width; ++c)
                y.at(i, c) = weightAt(tokenTable, (std::size_t) id * width + c)
                             + weightAt(positionTable, (std::size_t) (firstPosition + i) * width + c);
        }
        return keep(std::move(y));
    }

    Tensor appendLinear(Cache& cache, const Tensor& input, const Weight& weight, const Weight* bias) override
    {
        Storage& s = caches.at((std::size_t) cache.id);
        const Value y = project(of(input), weight, bias, Activation::none);
        if (y.cols != s.width || cache.rows + y.rows > s.capacity)
            throw std::logic_error("a cache was appended to past its capacity");
        std::copy(y.data.begin(), y.data.end(), s.data.begin() + (std::ptrdiff_t) cache.rows * s.width);
        cache.rows += y.rows;
        return cached(cache);
    }

    Cache makeCache(int capacityRows, int width) override
    {
        caches.push_back({capacityRows, width, std::vector<double>((std::size_t) capacityRows * width)});
        Cache c;
        c.id = (int) caches.size() - 1;
        return c;
    }

protected:
    void retain(int index) override { ++values.at((std::size_t) index).references; }
    void release(int index) override
    {
        Value& v = values.at((std::size_t) index);
        if (--v.references == 0)
            v.data.clear();
    }

private:
    struct Value
    {
        Value() = default;
        Value(int r, int c) : rows(r), cols(c), data((std::size_t) r * c) {}
        double& at(int r, int c) { return data[(std::size_t) r * cols + c]; }
        double at(int r, int c) const { return data[(std::size_t) r * cols + c]; }
        int rows = 0, cols = 0, references = 0;
        std::vector<double> data;
    };
    struct Storage
    {
        int capacity, width;
        std::vector<double> data;
    };

    static double weightAt(const Weight& w, std::size_t i)
    {
        const char* base = static_cast<const char*>(w.data());
        if (w.type == WeightStorage::Float)
        {
            float x;
            std::memcpy(&x, base + 4 * i, 4);
            return x;
        }
        std::uint16_t bits;
        std::memcpy(&bits, base + 2 * i, 2);
        if (w.type == WeightStorage::PackedBFloat16)
        {
            const std::uint32_t u = (std::uint32_t) bits << 16;
            float x;
            std::memcpy(&x, &u, 4);
            return x;
        }
        const int sign = bits >> 15, exponent = (bits >> 10) & 31, mantissa = bits & 1023;
        const double magnitude = exponent == 0    ? std::ldexp((double) mantissa, -24)
                                 : exponent == 31 ? (mantissa ? NAN : INFINITY)
                                                  : std::ldexp(1024.0 + mantissa, exponent - 25);
        return sign ? -magnitude : magnitude;
    }

    Value project(const Value& x, const Weight& weight, const Weight* bias, Activation activation) const
    {
        const int out = weight.dimension(0), inner = weight.dimension(1);
        if (x.cols != inner)
            throw std::logic_error("a projection's input width differs from its weight's");
        Value y(x.rows, out);
        for (int r = 0; r < x.rows; ++r)
            for (int o = 0; o < out; ++o)
            {
                double acc = 0;
                for (int k = 0; k < inner; ++k)
                    acc += x.at(r, k) * weightAt(weight, (std::size_t) o * inner + k);
                if (bias != nullptr)
                    acc += weightAt(*bias, (std::size_t) o);
                if (activation == Activation::gelu)
                    acc = 0.5 * acc * (1.0 + std::erf(acc / std::sqrt(2.0)));
                y.at(r, o) = acc;
            }
        return y;
    }

    const Value& of(const Tensor& t) const
    {
        if (!t.isOwnedBy(*this))
            throw std::logic_error("a tensor of another net");
        return values.at((std::size_t) t.index());
    }

    Tensor keep(Value v)
    {
        values.push_back(std::move(v));
        return Tensor(*this, (int) values.size() - 1);
    }

    std::vector<Value> values;
    std::vector<Storage> caches;
};
} // namespace WSP::Testing
