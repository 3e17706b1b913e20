// The safetensors reader, the config.json decoder shape and decoding fields, and
// the special tokens of a tokenizer.json (the JSON reader is json.h).
#include "../../../include/whispereacp/SafeTensors.h"
#include "../../../include/whispereacp/ModelError.h"
#include "host_common.h"
#include "json.h"

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <fcntl.h>
#include <fstream>
#include <limits>
#include <sstream>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <utility>

namespace WSP
{
namespace
{
// ---------------------------------------------------------------------------
// dtypes
// ---------------------------------------------------------------------------
struct TypeName
{
    const char* name;
    TensorType type;
    int bytes;
};

constexpr TypeName kTypes[] = {
    {"BOOL", TensorType::Bool, 1}, {"U8", TensorType::U8, 1},   {"I8", TensorType::I8, 1},
    {"U16", TensorType::U16, 2},   {"I16", TensorType::I16, 2}, {"F16", TensorType::F16, 2},
    {"BF16", TensorType::BF16, 2}, {"U32", TensorType::U32, 4}, {"I32", TensorType::I32, 4},
    {"F32", TensorType::F32, 4},   {"U64", TensorType::U64, 8}, {"I64", TensorType::I64, 8},
    {"F64", TensorType::F64, 8},
};

std::string describeShape(const std::vector<long long>& shape)
{
    std::ostringstream s;
    s << "[";
    for (std::size_t i = 0; i < shape.size(); ++i)
        s << (i ? "," : "") << shape[i];
    s << "]";
    return s.str();
}

std::uint64_t readLittleEndian64(const std::uint8_t* p)
{
    std::uint64_t v = 0;
    for (int i = 7; i >= 0; --i)
        v = (v << 8) | p[i];
    return v;
}
} // namespace

const char* tensorTypeName(TensorType type)
{
    for (const auto& t: kTypes)
        if (t.type == type)
            return t.name;
    return "?";
}

int tensorTypeBytes(TensorType type)
{
    for (const auto& t: kTypes)
        if (t.type == type)
            return t.bytes;
    return 0;
}

long long TensorInfo::elementCount() const
{
    long long n = 1;
    for (long long d: shape)
        n *= d;
    return n;
}

// Either a private copy of the bytes or a read-only mapping of the file.
struct SafeTensors::Storage
{
    std::vector<std::uint8_t> copy;
    void* map = nullptr;
    std::size_t mapBytes = 0;

    ~Storage()
    {
        if (map != nullptr)
            munmap(map, mapBytes);
    }
};

SafeTensors::SafeTensors(SafeTensors&&) noexcept = default;
SafeTensors& SafeTensors::operator=(SafeTensors&&) noexcept = default;
SafeTensors::~SafeTensors() = default;

SafeTensors SafeTensors::fromBytes(const void* bytes, std::size_t size)
{
    SafeTensors file;
    file.storage = std::make_unique<Storage>();
    file.storage->copy.assign(static_cast<const std::uint8_t*>(bytes), static_cast<const std::uint8_t*>(bytes) + size);
    file.parse(file.storage->copy.data(), size);
    return file;
}

SafeTensors SafeTensors::fromFile(const std::string& path)
{
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0)
        throw ModelError("cannot open '" + path + "': " + std::strerror(errno));
    struct stat st {};
    if (::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode))
    {
        ::close(fd);
        throw ModelError("'" + path + "' is not a regular file");
    }
    const std::size_t size = (std::size_t) st.st_size;
    SafeTensors file;
    file.storage = std::make_unique<Storage>();
    if (size > 0)
    {
        void* map = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (map == MAP_FAILED)
            throw ModelError("cannot map '" + path + "': " + std::strerror(errno));
        file.storage->map = map;
        file.storage->mapBytes = size;
        file.parse(static_cast<const std::uint8_t*>(map), size);
    }
    else
    {
        ::close(fd);
        file.parse(nullptr, 0);
    }
    return file;
}

void SafeTensors::parse(const std::uint8_t* bytes, std::size_t size)
{
    if (size < 8)
        throw ModelError("a safetensors file is shorter than its 8-byte header length");
    const std::uint64_t headerBytes = readLittleEndian64(bytes);
    if (headerBytes > size - 8)
        throw ModelError("the safetensors header length " + std::to_string(headerBytes) + " runs past the "
                         + std::to_string(size) + "-byte file");
    const char* text = reinterpret_cast<const char*>(bytes + 8);
    const Json header = JsonReader(text, text + headerBytes, "the safetensors header").document();
    if (header.kind != Json::Kind::Object)
        throw ModelError("the safetensors header is not a JSON object");
    blob = bytes + 8 + headerBytes;
    blobBytes = size - 8 - headerBytes;

    for (const auto& [key, value]: header.members)
    {
        if (key == "__metadata__")
        {
            if (value.kind != Json::Kind::Object)
                throw ModelError("__metadata__ is not an object");
            for (const auto& [mk, mv]: value.members)
            {
                if (mv.kind != Json::Kind::String)
                    throw ModelError("__metadata__ entry '" + mk + "' is not a string");
                meta[mk] = mv.text;
            }
            continue;
        }
        if (value.kind != Json::Kind::Object)
            throw ModelError("tensor '" + key + "' is not described by an object");
        const Json* dtype = value.member("dtype");
        const Json* shape = value.member("shape");
        const Json* offsets = value.member("data_offsets");
        if (dtype == nullptr || shape == nullptr || offsets == nullptr)
            throw ModelError("tensor '" + key + "' lacks dtype, shape or data_offsets");
        if (dtype->kind != Json::Kind::String)
            throw ModelError("tensor '" + key + "' has a dtype that is not a string");

        TensorInfo t;
        t.name = key;
        int elementBytes = 0;
        for (const auto& ty: kTypes)
            if (dtype->text == ty.name)
            {
                t.type = ty.type;
                elementBytes = ty.bytes;
            }
        if (elementBytes == 0)
            throw ModelError("tensor '" + key + "' has the unsupported dtype '" + dtype->text + "'");

        if (shape->kind != Json::Kind::Array)
            throw ModelError("tensor '" + key + "' has a shape that is not an array");
        long double elements = 1;
        for (const Json& d: shape->items)
        {
            if (d.kind != Json::Kind::Number || !d.integral || d.integer < 0)
                throw ModelError("tensor '" + key + "' has a shape entry that is not a non-negative integer");
            t.shape.push_back(d.integer);
            elements *= (long double) d.integer;
        }

        if (offsets->kind != Json::Kind::Array || offsets->items.size() != 2)
            throw ModelError("tensor '" + key + "' needs data_offsets [begin, end]");
        for (const Json& o: offsets->items)
            if (o.kind != Json::Kind::Number || !o.integral || o.integer < 0)
                throw ModelError("tensor '" + key + "' has a data offset that is not a non-negative integer");
        t.begin = (std::uint64_t) offsets->items[0].integer;
        t.end = (std::uint64_t) offsets->items[1].integer;
        if (t.end < t.begin)
            throw ModelError("tensor '" + key + "' ends before it begins");
        if (t.end > blobBytes)
            throw ModelError("tensor '" + key + "' runs past the " + std::to_string(blobBytes) + "-byte data blob");
        t.byteCount = t.end - t.begin;
        if ((long double) t.byteCount != elements * (long double) elementBytes)
            throw ModelError("tensor '" + key + "' has shape " + describeShape(t.shape) + " of " + dtype->text
                             + ", which is not the " + std::to_string(t.byteCount) + " bytes its range holds");
        entries.push_back(std::move(t));
    }
    std::sort(entries.begin(), entries.end(), [](const TensorInfo& a, const TensorInfo& b) { return a.name < b.name; });
    for (std::size_t i = 1; i < entries.size(); ++i)
        if (entries[i].name == entries[i - 1].name)
            throw ModelError("tensor '" + entries[i].name + "' is listed twice");

    for (const TensorInfo& t: entries)
    {
        HostTensor h;
        h.dtype = tensorTypeName(t.type);
        h.extents = t.shape;
        h.data = blob + t.begin;
        hostTensors.emplace(t.name, std::move(h));
    }
}

std::vector<std::string> SafeTensors::names() const
{
    std::vector<std::string> out;
    out.reserve(entries.size());
    for (const TensorInfo& t: entries)
        out.push_back(t.name);
    return out;
}

const TensorInfo* SafeTensors::findInfo(const std::string& name) const
{
    const auto it = std::lower_bound(entries.begin(), entries.end(), name,
                                     [](const TensorInfo& t, const std::string& n) { return t.name < n; });
    return it != entries.end() && it->name == name ? &*it : nullptr;
}

const TensorInfo& SafeTensors::info(const std::string& name) const
{
    const TensorInfo* t = findInfo(name);
    if (t == nullptr)
        throw ModelError("the safetensors file has no tensor '" + name + "'");
    return *t;
}

const HostTensor* SafeTensors::find(const std::string& name) const
{
    const auto it = hostTensors.find(name);
    return it == hostTensors.end() ? nullptr : &it->second;
}

void SafeTensors::readFloats(const std::string& name, float* destination, std::size_t capacity) const
{
    const TensorInfo& t = info(name);
    const std::size_t n = (std::size_t) t.elementCount();
    if (capacity < n)
        throw ModelError("tensor '" + name + "' holds " + std::to_string(n) + " values, more than the "
                         + std::to_string(capacity) + " the destination takes");
    if (n == 0)
        return; // an empty tensor's destination may be null, which memcpy must not see
    const std::uint8_t* p = rawBytes(t);
    switch (t.type)
    {
        case TensorType::F32: std::memcpy(destination, p, n * 4); break;
        case TensorType::F16:
        case TensorType::BF16:
            for (std::size_t i = 0; i < n; ++i)
            {
                std::uint16_t bits;
                std::memcpy(&bits, p + 2 * i, 2);
                destination[i] = t.type == TensorType::F16 ? halfToFloat(bits) : bfloat16ToFloat(bits);
            }
            break;
        case TensorType::F64:
            for (std::size_t i = 0; i < n; ++i)
            {
                double v;
                std::memcpy(&v, p + 8 * i, 8);
                destination[i] = (float) v;
            }
            break;
        default:
            throw ModelError("tensor '" + name + "' is " + tensorTypeName(t.type) + ", not a floating-point type");
    }
}

std::vector<float> SafeTensors::readFloats(const std::string& name) const
{
    std::vector<float> out((std::size_t) info(name).elementCount());
    readFloats(name, out.data(), out.size());
    return out;
}

// ---------------------------------------------------------------------------
// config.json
// ---------------------------------------------------------------------------
namespace
{
int positiveField(const Json& config, const char* key)
{
    const Json* v = config.member(key);
    if (v == nullptr)
        throw ModelError(std::string("config.json has no '") + key + "'");
    if (v->kind != Json::Kind::Number || !v->integral || v->integer <= 0 || v->integer > std::numeric_limits<int>::max())
        throw ModelError(std::string("config.json '") + key + "' is not a positive integer");
    return (int) v->integer;
}
} // namespace

DecoderShape decoderShapeFromConfig(const std::string& json, int crossPositionCount)
{
    const Json config = JsonReader(json.data(), json.data() + json.size(), "config.json").document();
    if (config.kind != Json::Kind::Object)
        throw ModelError("config.json is not a JSON object");
    if (const Json* type = config.member("model_type"))
        if (type->kind != Json::Kind::String || type->text != "whisper")
            throw ModelError("config.json describes a '" + (type->kind == Json::Kind::String ? type->text : "?")
                             + "' model, not a whisper one");
    DecoderShape s;
    s.width = positiveField(config, "d_model");
    s.heads = positiveField(config, "decoder_attention_heads");
    s.layers = positiveField(config, "decoder_layers");
    s.feedForwardWidth = positiveField(config, "decoder_ffn_dim");
    s.vocabularySize = positiveField(config, "vocab_size");
    s.maxPositions = positiveField(config, "max_target_positions");
    const int source = positiveField(config, "max_source_positions");
    if (s.width % s.heads != 0)
        throw ModelError("config.json d_model does not divide into the decoder head count");
    if (crossPositionCount < 0)
        throw ModelError("a negative cross position count");
    s.crossPositions = crossPositionCount == 0 ? source : crossPositionCount;
    return s;
}

namespace
{
std::string readText(const std::string& path)
{
    std::ifstream in(path, std::ios::binary);
    if (!in)
        throw ModelError("cannot open '" + path + "'");
    std::ostringstream text;
    text << in.rdbuf();
    return text.str();
}

int optionalToken(const Json& config, const char* key)
{
    const Json* v = config.member(key);
    if (v == nullptr || v->kind == Json::Kind::Null)
        return -1;
    if (v->kind != Json::Kind::Number || !v->integral || v->integer < 0 || v->integer > std::numeric_limits<int>::max())
        throw ModelError(std::string("config.json '") + key + "' is not a token id");
    return (int) v->integer;
}

std::vector<int> tokenList(const Json& config, const char* key)
{
    std::vector<int> ids;
    const Json* v = config.member(key);
    if (v == nullptr || v->kind == Json::Kind::Null)
        return ids;
    if (v->kind != Json::Kind::Array)
        throw ModelError(std::string("config.json '") + key + "' is not a list of token ids");
    for (const Json& item: v->items)
    {
        if (item.kind != Json::Kind::Number || !item.integral || item.integer > std::numeric_limits<int>::max()
            || item.integer < std::numeric_limits<int>::min())
            throw ModelError(std::string("config.json '") + key + "' holds an entry that is not a token id");
        ids.push_back((int) item.integer);
    }
    return ids;
}
} // namespace

DecoderShape decoderShapeFromConfigFile(const std::string& path, int crossPositionCount)
{
    return decoderShapeFromConfig(readText(path), crossPositionCount);
}

DecodingConfig decodingConfigFromConfig(const std::string& json)
{
    const Json config = JsonReader(json.data(), json.data() + json.size(), "config.json").document();
    if (config.kind != Json::Kind::Object)
        throw ModelError("config.json is not a JSON object");
    DecodingConfig c;
    c.vocabularySize = positiveField(config, "vocab_size");
    c.suppressedTokens = tokenList(config, "suppress_tokens");
    c.initiallySuppressedTokens = tokenList(config, "begin_suppress_tokens");
    c.decoderStartToken = optionalToken(config, "decoder_start_token_id");
    c.endOfTextToken = optionalToken(config, "eos_token_id");
    return c;
}

DecodingConfig decodingConfigFromConfigFile(const std::string& path)
{
    return decodingConfigFromConfig(readText(path));
}

namespace
{
// The name inside `<|...|>`, or empty.
std::string specialName(const std::string& content)
{
    if (content.size() < 5 || content.compare(0, 2, "<|") != 0 || content.compare(content.size() - 2, 2, "|>") != 0)
        return {};
    return content.substr(2, content.size() - 4);
}

bool languageCode(const std::string& name)
{
    if (name.size() != 2 && name.size() != 3)
        return false;
    return std::all_of(name.begin(), name.end(), [](char c) { return c >= 'a' && c <= 'z'; });
}

// "12.34" as seconds: digits, one dot with digits on both sides, nothing else.
bool timestampSeconds(const std::string& name, float& seconds)
{
    const std::size_t dot = name.find('.');
    if (dot == std::string::npos || dot == 0 || dot + 1 == name.size() || name.find('.', dot + 1) != std::string::npos)
        return false;
    if (!std::all_of(name.begin(), name.end(), [](char c) { return c == '.' || (c >= '0' && c <= '9'); }))
        return false;
    double whole = 0, fraction = 0, scale = 1;
    for (std::size_t i = 0; i < dot; ++i)
        whole = whole * 10 + (name[i] - '0');
    for (std::size_t i = dot + 1; i < name.size(); ++i)
    {
        fraction = fraction * 10 + (name[i] - '0');
        scale *= 10;
    }
    seconds = (float) (whole + fraction / scale);
    return true;
}
} // namespace

bool SpecialTokens::isTimestamp(int token) const
{
    return firstTimestamp >= 0 && token >= firstTimestamp && token < firstTimestamp + timestampCount;
}

int SpecialTokens::timestampForSeconds(float seconds) const
{
    if (timestampCount == 0 || timestampInterval <= 0.0f)
        return -1;
    const long step = std::lround(seconds / timestampInterval);
    return step < 0 || step >= timestampCount ? -1 : firstTimestamp + (int) step;
}

float SpecialTokens::secondsForTimestamp(int token) const
{
    return isTimestamp(token) ? (float) (token - firstTimestamp) * timestampInterval : -1.0f;
}

int SpecialTokens::forLanguage(const std::string& code) const
{
    const auto it = languages.find(code);
    return it == languages.end() ? -1 : it->second;
}

SpecialTokens specialTokensFromTokenizerJson(const std::string& json)
{
    const Json root = JsonReader(json.data(), json.data() + json.size(), "tokenizer.json").document();
    if (root.kind != Json::Kind::Object)
        throw ModelError("tokenizer.json is not a JSON object");
    SpecialTokens t;
    const Json* added = root.member("added_tokens");
    if (added == nullptr || added->kind == Json::Kind::Null)
        return t;
    if (added->kind != Json::Kind::Array)
        throw ModelError("tokenizer.json 'added_tokens' is not a list");
    float firstSeconds = 0.0f, lastSeconds = 0.0f;
    int lastTimestamp = -1;
    for (const Json& entry: added->items)
    {
        const Json* id = entry.kind == Json::Kind::Object ? entry.member("id") : nullptr;
        const Json* content = entry.kind == Json::Kind::Object ? entry.member("content") : nullptr;
        if (id == nullptr || id->kind != Json::Kind::Number || !id->integral || id->integer < 0
            || id->integer > std::numeric_limits<int>::max())
            throw ModelError("tokenizer.json has an added token without a token id");
        if (content == nullptr || content->kind != Json::Kind::String)
            throw ModelError("tokenizer.json has an added token without its text");
        const int token = (int) id->integer;
        const std::string name = specialName(content->text);
        if (name.empty())
            continue;
        float seconds = 0.0f;
        if (timestampSeconds(name, seconds))
        {
            if (t.firstTimestamp < 0 || token < t.firstTimestamp)
            {
                t.firstTimestamp = token;
                firstSeconds = seconds;
            }
            if (token > lastTimestamp)
            {
                lastTimestamp = token;
                lastSeconds = seconds;
            }
            ++t.timestampCount;
            continue;
        }
        static const std::pair<const char*, int SpecialTokens::*> named[] = {
            {"endoftext", &SpecialTokens::endOfText},         {"startoftranscript", &SpecialTokens::startOfTranscript},
            {"startofprev", &SpecialTokens::startOfPrevious}, {"startoflm", &SpecialTokens::startOfLanguageModel},
            {"translate", &SpecialTokens::translate},         {"transcribe", &SpecialTokens::transcribe},
            {"notimestamps", &SpecialTokens::noTimestamps},   {"nospeech", &SpecialTokens::noSpeech},
            {"nocaptions", &SpecialTokens::noSpeech}};
        bool matched = false;
        for (const auto& [key, field]: named)
            if (name == key)
            {
                t.*field = token;
                matched = true;
            }
        if (!matched && languageCode(name))
            t.languages.emplace(name, token);
    }
    if (t.timestampCount > 1 && lastTimestamp > t.firstTimestamp)
        t.timestampInterval = (lastSeconds - firstSeconds) / (float) (lastTimestamp - t.firstTimestamp);
    return t;
}

SpecialTokens specialTokensFromTokenizerFile(const std::string& path)
{
    return specialTokensFromTokenizerJson(readText(path));
}

std::vector<int> transcriptPrompt(const DecodingConfig& config, const SpecialTokens& specials)
{
    const int start = config.decoderStartToken >= 0 ? config.decoderStartToken : specials.startOfTranscript;
    if (start < 0)
        throw ModelError("neither config.json nor tokenizer.json names <|startoftranscript|>");
    if (specials.noTimestamps < 0)
        throw ModelError("tokenizer.json names no <|notimestamps|> token");
    if (config.vocabularySize > 0 && (start >= config.vocabularySize || specials.noTimestamps >= config.vocabularySize))
        throw ModelError("the prompt's tokens lie outside the vocabulary");
    return {start, specials.noTimestamps};
}

void DecodingConfig::suppressionMasks(std::vector<float>& firstStep, std::vector<float>& laterSteps) const
{
    auto mark = [this](std::vector<float>& mask, const std::vector<int>& ids) {
        for (int id: ids)
        {
            if (id < 0 || id >= vocabularySize)
                throw ModelError("config.json suppresses token " + std::to_string(id)
                                 + ", which is outside the vocabulary");
            mask[(std::size_t) id] = 1.0f;
        }
    };
    laterSteps.assign((std::size_t) vocabularySize, 0.0f);
    mark(laterSteps, suppressedTokens);
    firstStep = laterSteps;
    mark(firstStep, initiallySuppressedTokens);
}
} // namespace WSP
