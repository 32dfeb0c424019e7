"""Wire schema of the detection service, built at run time (no protoc in this image).

Package `yolo`, service `Yolo` with the one unary method `Detect`: the message names, field
numbers, types and labels are the reference's contract (proto/yolo.proto:4-56), so a client
generated from that file talks to this server unchanged, and this module's messages decode
the reference server's responses.  proto3: repeated scalars are packed.
"""
from __future__ import annotations

from google.protobuf import descriptor_pb2, descriptor_pool, message_factory

SERVICE = "yolo.Yolo"
METHOD = "Detect"
FULL_METHOD = f"/{SERVICE}/{METHOD}"

_F = descriptor_pb2.FieldDescriptorProto
_OPT, _REP = _F.LABEL_OPTIONAL, _F.LABEL_REPEATED

# (message, [(number, name, type, label, message type or None)]) -- proto/yolo.proto:9-56
_MESSAGES = [
    ("DetectRequest", [(1, "image", _F.TYPE_BYTES, _OPT, None),
                       (2, "model", _F.TYPE_STRING, _OPT, None)]),
    ("Box", [(1, "x1", _F.TYPE_FLOAT, _OPT, None), (2, "y1", _F.TYPE_FLOAT, _OPT, None),
             (3, "x2", _F.TYPE_FLOAT, _OPT, None), (4, "y2", _F.TYPE_FLOAT, _OPT, None),
             (5, "score", _F.TYPE_FLOAT, _OPT, None), (6, "cls", _F.TYPE_INT32, _OPT, None)]),
    ("RBox", [(1, "cx", _F.TYPE_FLOAT, _OPT, None), (2, "cy", _F.TYPE_FLOAT, _OPT, None),
              (3, "w", _F.TYPE_FLOAT, _OPT, None), (4, "h", _F.TYPE_FLOAT, _OPT, None),
              (5, "angle", _F.TYPE_FLOAT, _OPT, None), (6, "score", _F.TYPE_FLOAT, _OPT, None),
              (7, "cls", _F.TYPE_INT32, _OPT, None)]),
    ("ClassProb", [(1, "id", _F.TYPE_INT32, _OPT, None), (2, "prob", _F.TYPE_FLOAT, _OPT, None)]),
    ("Mask", [(1, "rle", _F.TYPE_UINT32, _REP, None)]),
    ("DetectResponse", [(1, "boxes", _F.TYPE_MESSAGE, _REP, "Box"),
                        (2, "queue_ms", _F.TYPE_FLOAT, _OPT, None),
                        (3, "infer_ms", _F.TYPE_FLOAT, _OPT, None),
                        (4, "batch", _F.TYPE_INT32, _OPT, None),
                        (5, "task", _F.TYPE_STRING, _OPT, None),
                        (6, "rboxes", _F.TYPE_MESSAGE, _REP, "RBox"),
                        (7, "classes", _F.TYPE_MESSAGE, _REP, "ClassProb"),
                        (8, "masks", _F.TYPE_MESSAGE, _REP, "Mask"),
                        (9, "mask_h", _F.TYPE_UINT32, _OPT, None),
                        (10, "mask_w", _F.TYPE_UINT32, _OPT, None),
                        (11, "lb_scale", _F.TYPE_FLOAT, _OPT, None),
                        (12, "lb_top", _F.TYPE_INT32, _OPT, None),
                        (13, "lb_left", _F.TYPE_INT32, _OPT, None)]),
]


def _build():
    f = descriptor_pb2.FileDescriptorProto(name="yolo11_amd/yolo.proto", package="yolo", syntax="proto3")
    for name, fields in _MESSAGES:
        m = f.message_type.add(name=name)
        for num, fname, ftype, label, tname in fields:
            fd = m.field.add(name=fname, number=num, type=ftype, label=label, json_name=fname)
            if tname:
                fd.type_name = f".yolo.{tname}"
    svc = f.service.add(name="Yolo")
    svc.method.add(name=METHOD, input_type=".yolo.DetectRequest", output_type=".yolo.DetectResponse")
    pool = descriptor_pool.DescriptorPool()
    pool.Add(f)
    return {name: message_factory.GetMessageClass(pool.FindMessageTypeByName(f"yolo.{name}"))
            for name, _ in _MESSAGES}


_CLASSES = _build()
DetectRequest = _CLASSES["DetectRequest"]
DetectResponse = _CLASSES["DetectResponse"]
Box = _CLASSES["Box"]
RBox = _CLASSES["RBox"]
ClassProb = _CLASSES["ClassProb"]
Mask = _CLASSES["Mask"]
