// The greedy loop of Whisper::decodeTranscript (Whisper/Whisper.cpp:1186-1224,
// 1361-1443): step 0 opens the sequence, decodes the prompt and samples its
// last row under the first-step mask; step j decodes the slot step j-1
// sampled into and samples under the later-step mask. The sampled token never
// leaves the device on its way to the next step; the host reads each step's
// slot and the persistent step's watchdog word, written together into pinned
// memory by one small launch behind the step, after that step's event,
// stepsInFlight steps ahead. A step whose hand-over timed out left its slot
// unwritten, so its token is never used and the run ends in
// std::runtime_error (the word is cleared).
#include "../../../include/whispereacp/GreedyDecoder.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <stdexcept>
#include <string>

namespace WSP
{
GreedyDecoder::GreedyDecoder(Decoder& decoderToUse, const DecoderWeights& weightsToUse, const Device& device)
    : decoder(decoderToUse), weights(weightsToUse)
{
    const DecoderShape& shape = decoder.shape();
    sequenceTokens = DeviceBuffer(device, (std::size_t) (shape.maxPositions + 1) * sizeof(std::uint32_t));
    logitRows = DeviceBuffer(device, (std::size_t) shape.maxPositions * shape.vocabularySize * sizeof(float));
    checkHip(hipHostMalloc(reinterpret_cast<void**>(&hostReports), 2 * stepsInFlight * sizeof(int), 0),
             "hipHostMalloc");
    for (int i = 0; i < stepsInFlight; ++i)
    {
        hipEvent_t e = nullptr;
        checkHip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
        events.push_back(e);
    }
}

GreedyDecoder::~GreedyDecoder()
{
    for (void* e : events)
        (void) hipEventDestroy(static_cast<hipEvent_t>(e));
    if (hostReports != nullptr)
        (void) hipHostFree(hostReports);
}

GreedyRun GreedyDecoder::decode(Pass& pass, const BufferRange& encoderRows, int crossPositionCount,
                                const std::vector<int>& prompt, int maximumTokens, int endOfText,
                                const float* firstMask, const float* laterMask)
{
    const DecoderShape& shape = decoder.shape();
    const int promptLength = (int) prompt.size();
    if (promptLength <= 0 || promptLength > shape.maxPositions)
        throw ModelError("a transcript needs a prompt of 1 to " + std::to_string(shape.maxPositions) + " tokens");
    if (maximumTokens <= 0)
        throw ModelError("a transcript has to be allowed at least one token");
    for (int id : prompt)
        if (id < 0 || id >= shape.vocabularySize)
            throw ModelError("prompt token " + std::to_string(id) + " is outside the vocabulary");

    const auto stream = static_cast<hipStream_t>(pass.hipStream());
    wsp_hip_ctx* const context = decoder.net().context();
    const int stepLimit = std::min(maximumTokens, shape.maxPositions - promptLength + 1);
    const std::size_t slotBytes = sizeof(std::uint32_t);
    const std::size_t rowBytes = (std::size_t) shape.vocabularySize * sizeof(float);
    auto slot = [&](int index) {
        return BufferRange {sequenceTokens.data(), (std::size_t) index * slotBytes, slotBytes};
    };

    std::vector<std::uint32_t> ids(prompt.begin(), prompt.end());
    checkHip(hipMemcpyAsync(sequenceTokens.data(), ids.data(), ids.size() * slotBytes, hipMemcpyHostToDevice, stream),
             "upload prompt");
    checkHip(hipStreamSynchronize(stream), "upload prompt");

    auto startStep = [&](int step) {
        const int target = promptLength + step;
        // The sampling step reports its token and watchdog word itself (a
        // persistent step; else the report below launches); a step that
        // trips writes nothing and leaves the nonzero word.
        int* pair = &hostReports[2 * (step % stepsInFlight)];
        pair[1] = -1;
        if (wsp_hip_step_report_next(context, pair) != WSP_OK)
            throw std::runtime_error(std::string("arm the step's report: ") + wsp_hip_last_error(context));
        if (step == 0)
        {
            // The prompt but its last token, then the last token with the
            // first step's sampling fused in: the same rows and the same token
            // as the whole prompt followed by an argmax of its last row.
            decoder.beginSequence(pass, encoderRows, weights, crossPositionCount);
            if (promptLength > 1)
                decoder.step(pass, BufferRange {sequenceTokens.data(), 0, (std::size_t) (promptLength - 1) * slotBytes},
                             promptLength - 1, weights, BufferRange::of(logitRows));
            decoder.stepAndSample(pass, slot(promptLength - 1), weights,
                                  BufferRange {logitRows.data(), (std::size_t) (promptLength - 1) * rowBytes, rowBytes},
                                  firstMask, slot(target));
        }
        else
            decoder.stepAndSample(pass, slot(target - 1), weights, BufferRange::of(logitRows), laterMask, slot(target));
        // The token and the watchdog word: written by the step itself, or in
        // one launch behind it.
        const int reported = wsp_hip_step_report(context, static_cast<const std::uint32_t*>(slot(target).data()),
                                                 pair);
        if (reported != WSP_OK)
            throw std::runtime_error(std::string("report the step's token: ") + wsp_hip_last_error(context));
        checkHip(hipEventRecord(static_cast<hipEvent_t>(events[(std::size_t) (step % stepsInFlight)]), stream),
                 "hipEventRecord");
    };

    GreedyRun run;
    const auto start = std::chrono::steady_clock::now();
    int nextStep = 0;
    while (nextStep < stepsInFlight && nextStep < stepLimit)
        startStep(nextStep++);

    for (int step = 0; step < nextStep; ++step)
    {
        checkHip(hipEventSynchronize(static_cast<hipEvent_t>(events[(std::size_t) (step % stepsInFlight)])),
                 "hipEventSynchronize");
        const int* report = &hostReports[2 * (step % stepsInFlight)];
        if (report[1] != 0)
        {
            // Drain what is in flight, then clear the word for the next run.
            (void) hipStreamSynchronize(stream);
            int status = 0;
            (void) wsp_hip_device_status(context, &status, 1);
            throw std::runtime_error("greedy decode: step " + std::to_string(step)
                                     + " timed out on the device (its hand-over watchdog tripped)");
        }
        const int sampled = report[0];
        ++run.steps;
        if (sampled == endOfText)
            break;
        run.tokens.push_back(sampled);
        if (nextStep < stepLimit)
            startStep(nextStep++);
    }
    run.decodeSeconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
    checkHip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    // Steps still in flight when end-of-text arrived have drained now; their
    // tokens are dropped, but a trip among them is reported, and the word is
    // left clear for the next run.
    int drained = 0;
    if (wsp_hip_device_status(context, &drained, 1) != WSP_OK)
        throw std::runtime_error(std::string("read the watchdog word: ") + wsp_hip_last_error(context));
    if (drained != 0)
        throw std::runtime_error("greedy decode: a step in flight after end-of-text timed out on the device (its "
                                 "hand-over watchdog tripped)");
    return run;
}
} // namespace WSP
