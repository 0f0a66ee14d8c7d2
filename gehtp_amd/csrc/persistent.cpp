// persistent.cpp — gehtp_persistent: a resident decode server over a file queue.
//
// The request/response protocol of the reference's device-resident runner
// (kernels/examples/42_gehtp_persistent/main.c:14-31, driven by
// scripts/persistent_runtime.py:1-17), served by a local process on the GPU host:
// the blob is parsed and its weights made resident once, KV states persist across
// requests, and each request is one wt_exec_run_io.
//
//   job file ("key value" lines, main.c:23-28):
//     blob <.wtop path>   out_temp <temp id>   in_bytes <run body bytes>
//     req <path>   resp <path>   out <path>   idle_exit_s <s, 0 = never; default 600>
//     weights_size <bytes of <blob stem>.weights.bin, optional>   trace <0|1>
//   request file: 4-byte big-endian header length, JSON header, then for op "run"
//     exactly in_bytes of input. Header keys: "op" (run|reset|ping|shutdown),
//     "want_out" (1: also write the out temp's bytes to the `out` path).
//   response file: 4-byte big-endian length + JSON:
//     run      {"rc":0,"token":t,"steps":n,"step_us":u}  (t = first max of the out
//              temp read as f16, main.c:345-347) or {"rc":<wt_exec rc>,"err":"..."}
//     ping     {"rc":0,"pong":1}     reset {"rc":0,"reset":1}     shutdown {"rc":0,"bye":1}
//     errors   {"rc":-1,"err":"bad_op" | "short_body" | "req_oversize" | ...}
//
// Differences from the device runner: the request is claimed (unlinked) once its
// size matches the frame, as there; the response is written to a temporary name and
// renamed, so a reader never sees a partial file. Usage: gehtp_persistent <job file>.
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "oplist_exec.h"
#include "oplist_parse.h"

namespace {

using Clock = std::chrono::steady_clock;

constexpr int kPollUs = 2000;                // request poll interval (main.c:53)
constexpr int64_t kFrameWaitUs = 5000000;    // wait for a growing request (main.c:54)

bool read_file(const std::string& p, std::vector<uint8_t>& out, size_t want = 0) {
    FILE* f = std::fopen(p.c_str(), "rb");
    if (!f) return false;
    if (!want) {
        std::fseek(f, 0, SEEK_END);
        const long sz = std::ftell(f);
        std::fseek(f, 0, SEEK_SET);
        if (sz <= 0) { std::fclose(f); return false; }
        want = (size_t)sz;
    }
    out.resize(want);
    const size_t got = std::fread(out.data(), 1, want, f);
    std::fclose(f);
    return got == want;
}

// "key value" line lookup (main.c:98-113).
bool job_get(const std::string& job, const char* key, std::string& out) {
    const size_t klen = std::strlen(key);
    size_t p = 0;
    while (p < job.size()) {
        size_t eol = job.find('\n', p);
        if (eol == std::string::npos) eol = job.size();
        if (eol - p > klen + 1 && job.compare(p, klen, key) == 0 && job[p + klen] == ' ') {
            out = job.substr(p + klen + 1, eol - p - klen - 1);
            while (!out.empty() && (out.back() == '\r' || out.back() == ' ')) out.pop_back();
            return true;
        }
        p = eol + 1;
    }
    return false;
}

// Minimal JSON value lookup for the flat headers the client writes (key order free).
bool json_str(const std::string& hdr, const char* key, std::string& v) {
    const std::string pat = std::string("\"") + key + "\"";
    size_t p = hdr.find(pat);
    if (p == std::string::npos) return false;
    p = hdr.find(':', p + pat.size());
    if (p == std::string::npos) return false;
    const size_t s = hdr.find('"', p);
    if (s == std::string::npos) return false;
    const size_t e = hdr.find('"', s + 1);
    if (e == std::string::npos) return false;
    v = hdr.substr(s + 1, e - s - 1);
    return true;
}

bool json_int(const std::string& hdr, const char* key, long& v) {
    const std::string pat = std::string("\"") + key + "\"";
    size_t p = hdr.find(pat);
    if (p == std::string::npos) return false;
    p = hdr.find(':', p + pat.size());
    if (p == std::string::npos) return false;
    char* end = nullptr;
    v = std::strtol(hdr.c_str() + p + 1, &end, 10);
    return end != hdr.c_str() + p + 1;
}

std::string json_escape(const char* s) {
    std::string o;
    for (; *s; ++s) {
        if (*s == '"' || *s == '\\') o += '\\';
        if ((unsigned char)*s < 0x20) { o += ' '; continue; }
        o += *s;
    }
    return o;
}

void write_resp(const std::string& path, const std::string& json) {
    const std::string tmp = path + ".tmp";
    FILE* f = std::fopen(tmp.c_str(), "wb");
    if (!f) return;
    const uint32_t n = (uint32_t)json.size();
    const uint8_t be[4] = {(uint8_t)(n >> 24), (uint8_t)(n >> 16), (uint8_t)(n >> 8), (uint8_t)n};
    std::fwrite(be, 1, 4, f);
    std::fwrite(json.data(), 1, json.size(), f);
    std::fclose(f);
    std::rename(tmp.c_str(), path.c_str());
}

int64_t file_size(const std::string& p) {
    struct stat st;
    return stat(p.c_str(), &st) == 0 ? (int64_t)st.st_size : -1;
}

// 1: no request; 0: a whole request in `req`; -1: a malformed request (answered).
int take_request(const std::string& req_p, const std::string& resp_p, uint32_t in_bytes,
                 std::vector<uint8_t>& req) {
    if (file_size(req_p) < 4) return 1;
    const auto t0 = Clock::now();
    auto waited_out = [&] {
        return std::chrono::duration_cast<std::chrono::microseconds>(Clock::now() - t0).count() > kFrameWaitUs;
    };
    // header length, then the header, then (for "run") the body: wait for each to land
    std::vector<uint8_t> head;
    for (;;) {
        if (read_file(req_p, head, 4)) break;
        if (waited_out()) { std::remove(req_p.c_str()); write_resp(resp_p, "{\"rc\":-1,\"err\":\"req_timeout\"}"); return -1; }
        std::this_thread::sleep_for(std::chrono::microseconds(kPollUs));
    }
    const uint32_t hl = ((uint32_t)head[0] << 24) | ((uint32_t)head[1] << 16) | ((uint32_t)head[2] << 8) | head[3];
    if (hl == 0 || hl > (1u << 20)) {
        std::remove(req_p.c_str());
        write_resp(resp_p, "{\"rc\":-1,\"err\":\"hdr_len_bad\"}");
        return -1;
    }
    size_t want = 4u + hl;
    for (;;) {
        if (file_size(req_p) >= (int64_t)want && read_file(req_p, head, want)) break;
        if (waited_out()) { std::remove(req_p.c_str()); write_resp(resp_p, "{\"rc\":-1,\"err\":\"hdr_read_fail\"}"); return -1; }
        std::this_thread::sleep_for(std::chrono::microseconds(kPollUs));
    }
    std::string op;
    if (json_str(std::string(head.begin() + 4, head.end()), "op", op) && op == "run") want += in_bytes;
    for (;;) {
        const int64_t sz = file_size(req_p);
        if (sz == (int64_t)want && read_file(req_p, req, want)) {
            std::remove(req_p.c_str());   // claimed: the client sees the file vanish
            return 0;
        }
        if (sz > (int64_t)want) {
            std::remove(req_p.c_str());
            write_resp(resp_p, "{\"rc\":-1,\"err\":\"req_oversize\"}");
            return -1;
        }
        if (waited_out()) { std::remove(req_p.c_str()); write_resp(resp_p, "{\"rc\":-1,\"err\":\"body_timeout\"}"); return -1; }
        std::this_thread::sleep_for(std::chrono::microseconds(kPollUs));
    }
}

// First strict maximum of the temp read as f16 (the reference runner's host argmax).
int32_t argmax_f16(const uint8_t* p, uint32_t bytes) {
    if (!p || bytes < 2) return -1;
    auto key = [](uint16_t h) -> float {
        const uint32_t s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
        float v;
        if (e == 0) v = std::ldexp((float)m, -24);
        else if (e == 31) v = m ? NAN : INFINITY;
        else v = std::ldexp((float)(m | 1024), (int)e - 25);
        return s ? -v : v;
    };
    int32_t best = 0;
    uint16_t h0;
    std::memcpy(&h0, p, 2);
    float bv = key(h0);
    for (uint32_t i = 1; i < bytes / 2; ++i) {
        uint16_t h;
        std::memcpy(&h, p + 2 * i, 2);
        const float v = key(h);
        if (v > bv) { bv = v; best = (int32_t)i; }
    }
    return best;
}

struct Server {
    wt_blob* w = nullptr;
    uint32_t out_temp = 0, in_bytes = 0, steps = 0;
    std::string resp_p, out_p;
};

// Returns true on shutdown (main.c:302-382).
bool handle(Server& sv, const std::vector<uint8_t>& req) {
    const uint32_t hl = ((uint32_t)req[0] << 24) | ((uint32_t)req[1] << 16) | ((uint32_t)req[2] << 8) | req[3];
    const std::string hdr(req.begin() + 4, req.begin() + 4 + hl);
    std::string op;
    const bool have_op = json_str(hdr, "op", op);
    long want_out = 0;
    json_int(hdr, "want_out", want_out);
    if (have_op && op == "ping") { write_resp(sv.resp_p, "{\"rc\":0,\"pong\":1}"); return false; }
    if (have_op && op == "reset") {
        wt_exec_state_reset();
        write_resp(sv.resp_p, "{\"rc\":0,\"reset\":1}");
        return false;
    }
    if (have_op && op == "shutdown") { write_resp(sv.resp_p, "{\"rc\":0,\"bye\":1}"); return true; }
    if (!have_op || op != "run") { write_resp(sv.resp_p, "{\"rc\":-1,\"err\":\"bad_op\"}"); return false; }
    const size_t body_off = 4u + hl;
    if (req.size() < body_off + sv.in_bytes) {
        write_resp(sv.resp_p, "{\"rc\":-1,\"err\":\"short_body\"}");
        return false;
    }
    char err[256] = {0};
    const auto t0 = Clock::now();
    const int rc = wt_exec_run_io(sv.w, req.data() + body_off, nullptr, sv.out_temp, nullptr, nullptr, err, sizeof err);
    const long long us = (long long)std::chrono::duration_cast<std::chrono::microseconds>(Clock::now() - t0).count();
    char resp[512];
    if (rc != 0) {
        std::snprintf(resp, sizeof resp, "{\"rc\":%d,\"err\":\"%s\"}", rc, json_escape(err).c_str());
    } else {
        const uint32_t nb = wt_exec_temp_last_bytes(sv.out_temp);
        const uint8_t* host = wt_exec_temp(sv.out_temp);
        if (!host || nb < 2) {
            // never written by this blob, or an intermediate a fused chain skipped
            write_resp(sv.resp_p, "{\"rc\":-1,\"err\":\"out_temp unavailable\"}");
            return false;
        }
        const int32_t tok = argmax_f16(host, nb);
        if (want_out) {
            const std::string tmp = sv.out_p + ".tmp";
            if (FILE* f = std::fopen(tmp.c_str(), "wb")) {
                std::fwrite(host, 1, nb, f);
                std::fclose(f);
                std::rename(tmp.c_str(), sv.out_p.c_str());
            }
        }
        ++sv.steps;
        std::snprintf(resp, sizeof resp, "{\"rc\":0,\"token\":%d,\"steps\":%u,\"step_us\":%lld}", (int)tok,
                      sv.steps, us);
    }
    write_resp(sv.resp_p, resp);
    return false;
}

}  // namespace

int main(int argc, char** argv) {
    const char* job_path = argc > 1 ? argv[1] : std::getenv("GEHTP_JOB");
    if (!job_path) {
        std::fprintf(stderr, "usage: gehtp_persistent <job file>\n");
        return 2;
    }
    std::vector<uint8_t> jb;
    if (!read_file(job_path, jb)) {
        std::fprintf(stderr, "[FAIL] read %s\n", job_path);
        return 1;
    }
    const std::string job(jb.begin(), jb.end());
    std::string blob_p, req_p, out_s, in_s, idle_s, wsz_s, trace_s;
    Server sv;
    if (!job_get(job, "blob", blob_p) || !job_get(job, "req", req_p) || !job_get(job, "resp", sv.resp_p) ||
        !job_get(job, "out", sv.out_p) || !job_get(job, "out_temp", out_s) || !job_get(job, "in_bytes", in_s)) {
        std::fprintf(stderr, "[FAIL] job file lacks a key (blob/req/resp/out/out_temp/in_bytes)\n");
        return 1;
    }
    sv.out_temp = (uint32_t)std::strtoul(out_s.c_str(), nullptr, 10);
    if (sv.out_temp >= WT_EXEC_MAX_TEMPS) {
        std::fprintf(stderr, "[FAIL] out_temp %u out of range (temps are 0..%u)\n", sv.out_temp, WT_EXEC_MAX_TEMPS - 1u);
        return 2;
    }
    sv.in_bytes = (uint32_t)std::strtoul(in_s.c_str(), nullptr, 10);
    const long idle_exit_s = job_get(job, "idle_exit_s", idle_s) ? std::strtol(idle_s.c_str(), nullptr, 10) : 600;
    const bool trace = job_get(job, "trace", trace_s) && std::strtol(trace_s.c_str(), nullptr, 10) != 0;
    std::remove(req_p.c_str());
    std::remove(sv.resp_p.c_str());

    std::vector<uint8_t> blob;
    if (!read_file(blob_p, blob)) {
        std::fprintf(stderr, "[FAIL] read blob %s\n", blob_p.c_str());
        return 1;
    }
    sv.w = static_cast<wt_blob*>(std::calloc(1, sizeof(wt_blob)));   // ~4.5 MB: heap, as the reference does
    if (!sv.w) return 1;
    const int prc = wt_parse(blob.data(), blob.size(), sv.w);
    if (prc != WT_OK) {
        std::fprintf(stderr, "[FAIL] wt_parse: %s\n", wt_err_str(prc));
        return 1;
    }
    wt_exec_set_trace(trace ? 1 : 0);
    std::vector<uint8_t> wgt;
    if (job_get(job, "weights_size", wsz_s)) {
        // <stem>.weights.bin next to the .wtop (main.c:441-460)
        std::string wp = blob_p;
        const size_t dot = wp.rfind('.');
        if (dot != std::string::npos && wp.compare(dot, std::string::npos, ".wtop") == 0) wp.erase(dot);
        wp += ".weights.bin";
        if (!read_file(wp, wgt, (size_t)std::strtoull(wsz_s.c_str(), nullptr, 10))) {
            std::fprintf(stderr, "[FAIL] ext weights read %s\n", wp.c_str());
            return 1;
        }
        wt_exec_set_ext_weights(wgt.data());
    }
    std::fprintf(stderr, "[ready] serving req=%s\n", req_p.c_str());

    auto t_last = Clock::now();
    bool stop = false;
    long served = 0;
    std::vector<uint8_t> req;
    while (!stop) {
        if (idle_exit_s > 0 && std::chrono::duration_cast<std::chrono::seconds>(Clock::now() - t_last).count() > idle_exit_s) {
            std::fprintf(stderr, "[idle] %lds without a request, exit\n", idle_exit_s);
            break;
        }
        const int r = take_request(req_p, sv.resp_p, sv.in_bytes, req);
        if (r == 0) {
            t_last = Clock::now();
            ++served;
            stop = handle(sv, req);
        } else if (r < 0) {
            t_last = Clock::now();
            ++served;
        } else {
            std::this_thread::sleep_for(std::chrono::microseconds(kPollUs));
        }
    }
    wt_exec_shutdown();
    std::free(sv.w);
    std::fprintf(stderr, "[stop] served %ld requests\n", served);
    return 0;
}
