"""A compact ResNet-50 (torchvision v1.5 layout: stride on the 3x3 conv of
each bottleneck) for the model-level checks; torchvision is not installed
here. Random initialisation only (no checkpoints): Kaiming-normal fan_out for
convolutions as torchvision does, BatchNorm weight 1 / bias 0, so a forward
in eval mode keeps activations at unit scale.

After ``replace_conv2d_with_nova`` 13 of its 3x3 convolutions run on the NOVA
path: 3 + 3 + 5 + 2 stride-1 bottleneck convs (64@56, 128@28, 256@14,
512@7); the first 3x3 of stages 2-4 has stride 2 and stays on MIOpen.
"""

import torch
import torch.nn as nn


class Bottleneck(nn.Module):
    expansion = 4

    def __init__(self, cin, width, stride=1, downsample=None):
        super().__init__()
        self.conv1 = nn.Conv2d(cin, width, 1, bias=False)
        self.bn1 = nn.BatchNorm2d(width)
        self.conv2 = nn.Conv2d(width, width, 3, stride=stride, padding=1, bias=False)
        self.bn2 = nn.BatchNorm2d(width)
        self.conv3 = nn.Conv2d(width, width * 4, 1, bias=False)
        self.bn3 = nn.BatchNorm2d(width * 4)
        self.relu = nn.ReLU(inplace=True)
        self.downsample = downsample

    def forward(self, x):
        idt = x if self.downsample is None else self.downsample(x)
        out = self.relu(self.bn1(self.conv1(x)))
        out = self.relu(self.bn2(self.conv2(out)))
        out = self.bn3(self.conv3(out))
        return self.relu(out + idt)


class ResNet50(nn.Module):
    def __init__(self, num_classes=1000):
        super().__init__()
        self.conv1 = nn.Conv2d(3, 64, 7, stride=2, padding=3, bias=False)
        self.bn1 = nn.BatchNorm2d(64)
        self.relu = nn.ReLU(inplace=True)
        self.maxpool = nn.MaxPool2d(3, stride=2, padding=1)
        layers, cin = [], 64
        for width, blocks, stride in ((64, 3, 1), (128, 4, 2), (256, 6, 2), (512, 3, 2)):
            ds = nn.Sequential(nn.Conv2d(cin, width * 4, 1, stride=stride, bias=False),
                               nn.BatchNorm2d(width * 4))
            stage = [Bottleneck(cin, width, stride, ds)]
            cin = width * 4
            stage += [Bottleneck(cin, width) for _ in range(blocks - 1)]
            layers.append(nn.Sequential(*stage))
        self.layer1, self.layer2, self.layer3, self.layer4 = layers
        self.avgpool = nn.AdaptiveAvgPool2d(1)
        self.fc = nn.Linear(2048, num_classes)
        for m in self.modules():
            if isinstance(m, nn.Conv2d):
                nn.init.kaiming_normal_(m.weight, mode="fan_out", nonlinearity="relu")
            elif isinstance(m, nn.BatchNorm2d):
                nn.init.ones_(m.weight)
                nn.init.zeros_(m.bias)

    def forward(self, x):
        x = self.maxpool(self.relu(self.bn1(self.conv1(x))))
        x = self.layer4(self.layer3(self.layer2(self.layer1(x))))
        return self.fc(torch.flatten(self.avgpool(x), 1))
